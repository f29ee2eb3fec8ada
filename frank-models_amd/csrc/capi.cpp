// C ABI of libfmoe.so: argument validation, workspace layout and the launch
// sequence of each entry point.  Declarations and reference citations are in
// include/fmoe.h (the kernel-path override for tests in include/fmoe_diag.h).
#include "fmoe.h"
#include "fmoe_diag.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "launch.h"

using namespace fmoe;

namespace {

thread_local char g_err[512] = "";
thread_local int g_last_path = FMOE_PATH_AUTO;
std::atomic<int> g_path{FMOE_PATH_AUTO};

constexpr int64_t kMaxExpert = 256;       // router lanes hold 4 experts each
constexpr int64_t kMaxExpertUsed = 64;    // one slot per lane in top-k
constexpr int64_t kMaxDim = (1ll << 31) - 1;
constexpr size_t kAlign = 256;

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return FMOE_OK;
}

#define FMOE_HIP(call)                                                                     \
  do {                                                                                     \
    hipError_t e_ = (call);                                                                \
    if (e_ != hipSuccess)                                                                  \
      return fail(FMOE_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_));            \
  } while (0)

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool act_dtype_ok(int dt) { return dt == FMOE_F32 || dt == FMOE_BF16; }
bool w_dtype_ok(int dt) { return dt == FMOE_F32 || dt == FMOE_BF16 || dt == FMOE_F8E4M3FN; }
// The block and sub-layer also take FMOE_F8E4M3FN_A8 and _A8X2: e4m3fn
// weights whose prefill GEMMs run on fp8 activations (one or two e4m3 terms).
bool fp8_act_dtype(int dt) { return dt == FMOE_F8E4M3FN_A8 || dt == FMOE_F8E4M3FN_A8X2; }
bool block_w_dtype_ok(int dt) { return w_dtype_ok(dt) || fp8_act_dtype(dt); }
// Storage type of the packed weights for a block weight dtype.
int packed_dtype(int dt) { return fp8_act_dtype(dt) ? FMOE_F8E4M3FN : dt; }

bool aligned_for(const void* p, int dt) {
  return reinterpret_cast<uintptr_t>(p) % dtype_bytes(dt) == 0;
}

// Device check, cached per device ordinal.
std::mutex g_dev_mu;
int g_dev_state[64] = {0};  // 0 unknown, 1 gfx950, -1 other

int ensure_device(int* dev_out = nullptr, char* arch = nullptr, size_t arch_len = 0) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(FMOE_ERR_NO_DEVICE, "no HIP device available (%s)",
                e == hipSuccess ? "device count 0" : hipGetErrorString(e));
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FMOE_ERR_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev_out) *dev_out = dev;
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if (dev < 64 && g_dev_state[dev] == 1 && !arch) return FMOE_OK;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess)
    return fail(FMOE_ERR_NO_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (arch && arch_len) {
    strncpy(arch, prop.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = '\0';
  }
  const bool is950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  if (dev < 64) g_dev_state[dev] = is950 ? 1 : -1;
  if (!is950)
    return fail(FMOE_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only", dev,
                prop.gcnArchName);
  return FMOE_OK;
}

// ------------------------------------------------------------ kernel timing
// Event pairs recorded around launches while timing is enabled; read back
// (and recycled) by fmoe_timing_read.
struct PendingTiming {
  int timer;
  hipEvent_t start, stop;
};

std::mutex g_t_mu;
std::atomic<bool> g_timing{false};
std::vector<PendingTiming> g_pending;
std::vector<hipEvent_t> g_event_pool;
double g_t_ms[FMOE_TIMER_COUNT] = {0};
int64_t g_t_calls[FMOE_TIMER_COUNT] = {0};

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  // Timing-only events: no system-scope release when recorded, so a record
  // neither writes back and invalidates the caches nor slows the launches
  // that follow (the readback waits on the event and reads its timestamps).
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

class ScopedTimer {
 public:
  ScopedTimer(int timer, hipStream_t s, bool allowed = true) : timer_(timer), s_(s) {
    if (!allowed || !g_timing.load(std::memory_order_relaxed)) return;
    std::lock_guard<std::mutex> lk(g_t_mu);
    start_ = take_event();
    stop_ = take_event();
    if (start_ && stop_) (void)hipEventRecord(start_, s_);
  }
  ~ScopedTimer() {
    if (!start_ || !stop_) return;
    (void)hipEventRecord(stop_, s_);
    std::lock_guard<std::mutex> lk(g_t_mu);
    g_pending.push_back({timer_, start_, stop_});
  }

 private:
  int timer_;
  hipStream_t s_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
};

// The kernel family (FMOE_PATH_*) and tiled variant run_grouped_gemm takes
// for g under the process-wide setting.
int pick_path(const GroupedGemmArgs& g, int* variant_out) {
  const int want = g_path.load(std::memory_order_relaxed);
  GroupedGemmArgs probe = g;
  probe.ksplit = 1;
  const bool can_tile = resolve_tiled_variant(probe, TILED_AUTO) >= 0;
  const bool can_stream = gemm_stream_supported(probe);
  int path = FMOE_PATH_GENERIC;
  int variant = TILED_AUTO;
  if (want == FMOE_PATH_TILED_LARGE && gemm_tiled256_supported(probe)) {
    path = FMOE_PATH_TILED_LARGE;
    variant = TILED_256;
  } else if ((want == FMOE_PATH_TILED || want == FMOE_PATH_TILED_LARGE) && can_tile) {
    path = FMOE_PATH_TILED;
    variant = want == FMOE_PATH_TILED ? TILED_128 : TILED_AUTO;
  } else if (want == FMOE_PATH_STREAM && can_stream) {
    path = FMOE_PATH_STREAM;
  } else if (want == FMOE_PATH_GENERIC) {
    path = FMOE_PATH_GENERIC;
  } else {
    // Few rows per expert (<= 8 on average): stream the weights once;
    // otherwise tile.  Measured crossover: at 8 rows per expert streaming
    // wins, at 16 the 256-tile kernel wins or ties (fp8 and skewed routing
    // clearly).
    const bool small = static_cast<int64_t>(g.n_assign) <= 8ll * g.n_expert;
    if (small && can_stream)
      path = FMOE_PATH_STREAM;
    else if (can_tile)
      path = FMOE_PATH_TILED;
    else if (can_stream)
      path = FMOE_PATH_STREAM;
  }
  if (path == FMOE_PATH_TILED || path == FMOE_PATH_TILED_LARGE) variant = resolve_tiled_variant(probe, variant);
  *variant_out = variant;
  return path;
}

// Runs one grouped GEMM on the family the process-wide setting asks for,
// falling back to the automatic choice when that family cannot run it.
// `g.split_stride` > 0 offers room for a K split into fp32 partials; the
// split used is returned in *ksplit_used (1 if none).
int run_grouped_gemm(GroupedGemmArgs g, hipStream_t s, int* ksplit_used = nullptr) {
  int variant = TILED_AUTO;
  const int path = pick_path(g, &variant);
  // Routing in the GEMM's blocks: only the streaming kernel computes it.
  if (g.rp.part && path != FMOE_PATH_STREAM)
    return fail(FMOE_ERR_HIP, "routed gate/up GEMM: the streaming kernel is not the chosen family");
  g.ksplit = 1;
  if ((path == FMOE_PATH_TILED || path == FMOE_PATH_TILED_LARGE) && variant == TILED_256 && g.split_stride > 0)
    g.ksplit = gemm_tiled256_ksplit(g);
  hipError_t e;
  if (path == FMOE_PATH_TILED || path == FMOE_PATH_TILED_LARGE)
    e = launch_gemm_tiled(g, s, variant);
  else if (path == FMOE_PATH_STREAM)
    e = launch_gemm_stream(g, s);
  else
    e = launch_gemm_generic(g, s);
  g_last_path = path;
  if (ksplit_used) *ksplit_used = g.ksplit;
  if (e != hipSuccess) return fail(FMOE_ERR_HIP, "grouped GEMM launch: %s", hipGetErrorString(e));
  return FMOE_OK;
}

// ------------------------------------------------------------ workspaces
struct PermuteLayout {
  size_t order, offsets, err, scratch, total;
};

PermuteLayout permute_layout(int64_t n_assign, int64_t n_expert, size_t base = 0) {
  PermuteLayout L;
  size_t off = base;
  L.err = off;
  off += align_up(16);
  L.scratch = off;  // chunk histograms of a large batch
  off += align_up(permute_scratch_bytes(static_cast<int>(n_assign), static_cast<int>(n_expert)));
  L.order = off;
  off += align_up(static_cast<size_t>(n_assign) * 4);
  L.offsets = off;
  off += align_up(static_cast<size_t>(n_expert + 1) * 4);
  L.total = off;
  return L;
}

struct MmidLayout {
  PermuteLayout perm;
  size_t x, y, total;
};

MmidLayout mmid_layout(int64_t n_out, int64_t n_in, int64_t n_expert, int64_t k, int64_t T,
                       int act) {
  MmidLayout L;
  const int64_t n = k * T;
  L.perm = permute_layout(n, n_expert);
  size_t off = L.perm.total;
  L.x = off;
  off += align_up(static_cast<size_t>(n) * n_in * dtype_bytes(act));
  L.y = off;
  off += align_up(static_cast<size_t>(n) * n_out * dtype_bytes(act));
  L.total = off;
  return L;
}

struct BlockLayout {
  size_t ids, weights;
  PermuteLayout perm;
  size_t h, y, total;
  size_t xkb, xkb_bytes;  // token rows gathered K-blocked in expert order (0 bytes when no prefill GEMM can use them)
  // fp8 activations (FMOE_F8E4M3FN_A8, prefill-sized batches): e4m3 token
  // rows and SwiGLU rows, K-blocked, with their per-row scales (0 bytes otherwise)
  size_t xq, xs, hq, hs, hmax, xmax, a8_bytes;
  // FMOE_F8E4M3FN_A8X2: bytes from the hi codes to the lo codes of x and h
  // (0 with one term)
  size_t x_plane, h_plane;
  size_t rpart;          // split router logits, decode or prefill (0 bytes when the shape takes the one-kernel router)
  size_t rpart_bytes;
  // tile schedules of the prefill GEMMs (256-tile kernel; 0 bytes when the shape takes none)
  size_t ttab_g, ttab_g_bytes, ttab_d, ttab_d_bytes;
  int h_dtype, y_dtype;
  int y_parts;           // fp32 partial buffers reserved for a K-split down GEMM
  int64_t y_part_elems;  // elements per partial
};

// Shape-only part of the down projection's GEMM arguments (the split
// decision depends on nothing else).
GroupedGemmArgs down_shape(int64_t T, int64_t E, int64_t k, int64_t H, int64_t F, int act, int wdt) {
  GroupedGemmArgs d;
  d.a_mode = A_DIRECT;
  d.lda = F;
  d.n_tokens = static_cast<int>(T);
  d.n_assign = static_cast<int>(T * k);
  d.n_expert = static_cast<int>(E);
  d.N = H;
  d.K = F;
  d.ldo = H;
  d.epi = EPI_SCATTER_WEIGHTED;
  d.act_dtype = act;
  d.w_dtype = wdt;
  d.w_format = packed_format(H, F, wdt);
  d.out_dtype = FMOE_F32;
  d.split_stride = 1;
  return d;
}

BlockLayout block_layout(int64_t T, int64_t E, int64_t k, int64_t H, int64_t F, int act, int block_wdt) {
  const int wdt = packed_dtype(block_wdt);
  BlockLayout L;
  const int64_t n = k * T;
  size_t off = 0;
  L.ids = off;
  off += align_up(static_cast<size_t>(n) * 4);
  L.weights = off;
  off += align_up(static_cast<size_t>(n) * 4);
  L.perm = permute_layout(n, E, off);
  off = L.perm.total;
  L.rpart = off;
  L.rpart_bytes = std::max(router_decode_scratch_bytes(static_cast<int>(T), static_cast<int>(H),
                                                       static_cast<int>(E), static_cast<int>(k), act),
                           router_prefill_scratch_bytes(static_cast<int>(T), static_cast<int>(H),
                                                        static_cast<int>(E), static_cast<int>(k), act));
  off += align_up(L.rpart_bytes);
  L.h_dtype = act;
  L.h = off;
  off += align_up(static_cast<size_t>(n) * F * dtype_bytes(L.h_dtype));
  L.y_dtype = FMOE_F32;
  L.y_part_elems = n * H;
  L.y_parts = (n > 0 && H > 0 && F > 0) ? gemm_tiled256_ksplit(down_shape(T, E, k, H, F, act, wdt)) : 1;
  L.y = off;
  off += align_up(static_cast<size_t>(n) * H * dtype_bytes(L.y_dtype) * L.y_parts);
  // Prefill-sized bf16 batches: room for the token rows gathered into expert
  // order, K-blocked, so the gate/up GEMM reads whole cache lines.
  const bool prefill = act == FMOE_BF16 && n > 8 * E;
  const bool a8 = prefill && fp8_act_dtype(block_wdt) && H % 128 == 0 && F % 128 == 0 && H <= 16384 &&
                  F <= 16384;
  const bool kb_candidate = prefill && !a8 && H % 64 == 0 && F % 64 == 0 && (F + 127) / 128 >= 16;
  L.ttab_g_bytes = 0;
  L.ttab_d_bytes = 0;
  if (prefill) {
    GroupedGemmArgs gs = down_shape(T, E, k, H, F, act, wdt);
    L.ttab_d_bytes = gemm_tiled256_table_bytes(gs);
    gs.epi = EPI_SWIGLU;
    gs.N = F;
    gs.K = H;
    gs.split_stride = 0;
    L.ttab_g_bytes = gemm_tiled256_table_bytes(gs);
  }
  L.ttab_g = off;
  off += align_up(L.ttab_g_bytes);
  L.ttab_d = off;
  off += align_up(L.ttab_d_bytes);
  L.xkb = off;
  L.xkb_bytes = kb_candidate ? static_cast<size_t>(n) * H * 2 : 0;
  off += align_up(L.xkb_bytes);
  L.a8_bytes = 0;
  L.x_plane = L.h_plane = 0;
  L.xq = off;
  if (a8) {
    const int terms = block_wdt == FMOE_F8E4M3FN_A8X2 ? 2 : 1;
    if (terms == 2) {
      L.x_plane = align_up(static_cast<size_t>(n) * H);
      L.h_plane = align_up(static_cast<size_t>(n) * F);
    }
    off += terms * align_up(static_cast<size_t>(n) * H);
    L.xs = off;
    off += align_up(static_cast<size_t>(n) * 4);
    L.hq = off;
    off += terms * align_up(static_cast<size_t>(n) * F);
    L.hs = off;
    off += align_up(static_cast<size_t>(n) * 4);
    L.hmax = off;
    off += align_up(static_cast<size_t>(n) * 4);
    L.xmax = off;
    off += align_up(static_cast<size_t>(T) * 4);
    L.a8_bytes = off - L.xq;
  } else {
    L.xs = L.hq = L.hs = L.hmax = L.xmax = off;
  }
  L.total = off;
  return L;
}

template <typename T>
T* at(void* base, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

int check_dims(const char* what, int64_t v, int64_t lo, int64_t hi) {
  if (v < lo || v > hi)
    return fail(FMOE_ERR_SHAPE, "%s=%lld outside [%lld, %lld]", what, static_cast<long long>(v),
                static_cast<long long>(lo), static_cast<long long>(hi));
  return FMOE_OK;
}

#define FMOE_TRY(x)            \
  do {                         \
    int r_ = (x);              \
    if (r_ != FMOE_OK) return r_; \
  } while (0)

int validate_router(int64_t T, int64_t H, int64_t E, int64_t k) {
  FMOE_TRY(check_dims("n_tokens", T, 0, kMaxDim));
  FMOE_TRY(check_dims("n_embd", H, 1, kMaxDim));
  FMOE_TRY(check_dims("n_expert", E, 1, kMaxExpert));
  FMOE_TRY(check_dims("n_expert_used", k, 1, E < kMaxExpertUsed ? E : kMaxExpertUsed));
  if (k * T > kMaxDim) return fail(FMOE_ERR_SHAPE, "n_expert_used * n_tokens exceeds 2^31-1");
  return FMOE_OK;
}

struct BlockCall {
  const void* input;
  const void* w_router;
  const void* packed_up;
  const void* packed_gate;
  const void* packed_down;
  const float* up_scales;
  const float* gate_scales;
  const float* down_scales;
  int w_dtype;
  void* out;
  const void* residual;  // added to the block output by combine (may be null)
  int64_t n_tokens, n_expert, n_expert_used, n_embd, n_ff;
  int normalize_weights;
  int act_dtype;
  void* workspace;
  size_t workspace_bytes;
  void* stream;
  bool timers = true;    // false: no timing events (the allocation-free entry point)
};

// The block's workspace followed by the normalised input rows.
struct SublayerLayout {
  BlockLayout block;
  size_t xn, total;
};

SublayerLayout sublayer_layout(int64_t T, int64_t E, int64_t k, int64_t H, int64_t F, int act, int wdt) {
  SublayerLayout SL;
  SL.block = block_layout(T, E, k, H, F, act, wdt);
  SL.xn = SL.block.total;
  SL.total = SL.xn + align_up(static_cast<size_t>(T) * H * dtype_bytes(act));
  return SL;
}

int check_workspace(const void* ws, size_t bytes, size_t need) {
  if (!ws) return fail(FMOE_ERR_INVALID_ARGUMENT, "null workspace");
  if (bytes < need) return fail(FMOE_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", bytes, need);
  if (reinterpret_cast<uintptr_t>(ws) % kAlign)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "workspace must be %zu-byte aligned", kAlign);
  return FMOE_OK;
}

// Argument checks shared by the block and the sub-layer (the reference
// checks none of these; moe_ffn_block.mlir:34-45 only declares the types).
int validate_block(const BlockCall& c) {
  if (!act_dtype_ok(c.act_dtype)) return fail(FMOE_ERR_DTYPE, "activation dtype %d", c.act_dtype);
  if (!block_w_dtype_ok(c.w_dtype)) return fail(FMOE_ERR_DTYPE, "weight dtype %d", c.w_dtype);
  if (c.act_dtype == FMOE_F32 && c.w_dtype != FMOE_F32)
    return fail(FMOE_ERR_DTYPE, "f32 activations need f32 weights");
  FMOE_TRY(validate_router(c.n_tokens, c.n_embd, c.n_expert, c.n_expert_used));
  FMOE_TRY(check_dims("n_ff", c.n_ff, 0, kMaxDim));
  if (c.normalize_weights != 0 && c.normalize_weights != 1)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "normalize_weights must be 0 or 1");
  if (c.n_tokens == 0) return FMOE_OK;
  if (!c.input || !c.w_router || !c.packed_up || !c.packed_gate || !c.packed_down || !c.out)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (packed_dtype(c.w_dtype) == FMOE_F8E4M3FN && (!c.up_scales || !c.gate_scales || !c.down_scales))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "fp8 weights need scales");
  if (!aligned_for(c.input, c.act_dtype) || !aligned_for(c.out, c.act_dtype) ||
      !aligned_for(c.w_router, c.act_dtype))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  return FMOE_OK;
}

// Prefill GEMMs on the 256-tile kernel take a per-launch tile schedule.
constexpr bool kTileTable = true;

// The MoE FFN block's kernel sequence (moe_ffn_block.mlir:47-208) on a
// validated call whose workspace holds layout L.
int run_block(const BlockCall& c, const BlockLayout& L) {
  hipStream_t s = static_cast<hipStream_t>(c.stream);
  void* workspace = c.workspace;
  const int64_t n_embd = c.n_embd, n_ff = c.n_ff, n_expert = c.n_expert, n_expert_used = c.n_expert_used;
  const int act_dtype = c.act_dtype, w_dtype = packed_dtype(c.w_dtype);
  const int T = static_cast<int>(c.n_tokens);
  const int n = static_cast<int>(c.n_tokens * n_expert_used);
  int* ids = at<int>(workspace, L.ids);
  float* rw = at<float>(workspace, L.weights);
  int* err = at<int>(workspace, L.perm.err);
  int* order = at<int>(workspace, L.perm.order);
  int* offsets = at<int>(workspace, L.perm.offsets);
  void* h = at<char>(workspace, L.h);
  void* y = at<char>(workspace, L.y);

  // Steps 1-4: router logits, softmax, top-k, renormalisation (mlir:50-128),
  // then the slot-major assignments grouped by expert (replaces the gather,
  // mul_mat_id.mlir:50-61).  Decode-sized batches run both as two launches,
  // or (at most 4 tokens) as the logits launch plus the gate/up GEMM's
  // blocks; the launches follow the GEMM setup below.
  const bool router16 = reinterpret_cast<uintptr_t>(c.input) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(c.w_router) % 16 == 0;
  const int H32 = static_cast<int>(n_embd), E32 = static_cast<int>(n_expert), k32 = static_cast<int>(n_expert_used);
  const bool decode_router = router16 && router_decode_scratch_bytes(T, H32, E32, k32, act_dtype) > 0 &&
                             L.rpart_bytes >= router_decode_scratch_bytes(T, H32, E32, k32, act_dtype);
  const bool split_router = router16 && !decode_router && router_prefill_scratch_bytes(T, H32, E32, k32, act_dtype) > 0 &&
                            L.rpart_bytes >= router_prefill_scratch_bytes(T, H32, E32, k32, act_dtype);

  // Steps 5-8: up and gate projections + SwiGLU (mlir:130-156), h[p, :] per sorted row p.
  GroupedGemmArgs g;
  g.a = c.input;
  g.lda = n_embd;
  g.a_mode = A_GATHER_TOKEN;
  g.order = order;
  g.offsets = offsets;
  g.n_tokens = T;
  g.n_assign = n;
  g.n_expert = static_cast<int>(n_expert);
  g.w0 = c.packed_gate;
  g.w1 = c.packed_up;
  if (w_dtype == FMOE_F8E4M3FN) {
    g.s0 = c.gate_scales;
    g.s1 = c.up_scales;
  }
  g.N = n_ff;
  g.K = n_embd;
  g.out = h;
  g.ldo = n_ff;
  g.epi = EPI_SWIGLU;
  g.act_dtype = act_dtype;
  g.w_dtype = w_dtype;
  g.w_format = packed_format(n_ff, n_embd, w_dtype);
  g.out_dtype = L.h_dtype;
  g.max_rows_per_expert = T;  // top-k experts are distinct per token
  GroupedGemmArgs d = down_shape(T, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype);
  d.a = h;
  d.order = order;
  d.offsets = offsets;
  d.w0 = c.packed_down;
  d.s0 = w_dtype == FMOE_F8E4M3FN ? c.down_scales : nullptr;
  d.out = y;
  d.route_w = rw;
  d.act_dtype = L.h_dtype;
  d.split_stride = L.y_parts > 1 ? L.y_part_elems : 0;
  d.max_rows_per_expert = T;

  // When both GEMMs take the 256-tile kernel, their A operands go K-blocked
  // (64-byte row pieces, one contiguous run per stage of a tile): the token
  // rows are gathered into expert order first, and the gate/up epilogue
  // writes h in that layout for the down GEMM.  With fp8 activations
  // (FMOE_F8E4M3FN_A8) the gathered rows and h are quantised to e4m3 per row
  // instead, and both GEMMs run on the fp8 MFMA.
  // The 256-tile down GEMM stores its weighted per-slot rows (and K-split
  // partials) in bf16, the activation type, halving the traffic of its
  // epilogue and of combine; the other paths keep fp32.
  // Only decisions here: the launches that read the permutation follow it.
  bool h_quant = false, gather_x = false;
  int y_dtype = L.y_dtype;
  GroupedGemmArgs dq = d;
  if (n > 8 * n_expert && act_dtype == FMOE_BF16) {
    int vg = 0, vd = 0;
    const int pg = pick_path(g, &vg), pd = pick_path(d, &vd);
    const bool tiled_g = pg == FMOE_PATH_TILED || pg == FMOE_PATH_TILED_LARGE;
    const bool tiled_d = pd == FMOE_PATH_TILED || pd == FMOE_PATH_TILED_LARGE;
    const bool both256 = tiled_g && tiled_d && vg == TILED_256 && vd == TILED_256;
    GroupedGemmArgs gk = g, dk = d;
    gk.a_mode = A_DIRECT;
    gk.a_kb_rows = n;
    dk.a_kb_rows = n;
    dk.out_dtype = FMOE_BF16;
    if (L.a8_bytes) {
      gk.a_lo_plane = static_cast<int64_t>(L.x_plane);
      dk.a_lo_plane = static_cast<int64_t>(L.h_plane);
      gk.a = at<char>(workspace, L.xq);
      gk.act_dtype = DT_F8;
      gk.a_scale = at<float>(workspace, L.xs);
      gk.row_amax = at<unsigned>(workspace, L.hmax);
      dk.a = at<char>(workspace, L.hq);
      dk.act_dtype = DT_F8;
      dk.a_scale = at<float>(workspace, L.hs);
      if (both256 && gemm_tiled256_supported(gk) && gemm_tiled256_supported(dk)) {
        g = gk;
        dq = dk;
        h_quant = true;
        y_dtype = FMOE_BF16;
      }
    } else {
      // h goes K-blocked at no cost; the token rows are worth gathering only
      // when many column tiles of the gate/up GEMM re-read them (measured:
      // Mixtral's 112 tiles gain 77 us for a 19 us gather, Qwen3's 6 tiles
      // lose 74 us at 8192 tokens).
      const bool want_gather = (n_ff + 127) / 128 >= 16;
      GroupedGemmArgs gh = g;  // gate/up reading the token rows in place
      gh.out_kb_rows = n;
      if (want_gather) {
        gk.a = at<char>(workspace, L.xkb);
        gk.out_kb_rows = n;
      }
      GroupedGemmArgs& gsel = want_gather ? gk : gh;
      if (both256 && gemm_tiled256_supported(gsel) && gemm_tiled256_supported(dk)) {
        gather_x = want_gather;
        g = gsel;
        d = dk;
        y_dtype = FMOE_BF16;
      }
    }
    // The 256-tile GEMMs deal their tiles from a per-launch schedule table
    // (ignored by the other kernel families), each in its reserved room,
    // built by the permutation below where there is one.
    if (kTileTable) {
      GroupedGemmArgs* dn = h_quant ? &dq : &d;
      const struct {
        GroupedGemmArgs* x;
        size_t at, bytes;
      } tabs[2] = {{&g, L.ttab_g, L.ttab_g_bytes}, {dn, L.ttab_d, L.ttab_d_bytes}};
      for (const auto& tb : tabs) {
        const size_t need = gemm_tiled256_table_bytes(*tb.x);
        if (need > 0 && need <= tb.bytes) tb.x->tile_table = at<int>(workspace, tb.at);
      }
    }
  }

  // The router.  Decode batches of at most 4 tokens (k * n_tokens <= 64)
  // whose gate/up GEMM takes the streaming kernel under the automatic choice
  // run their softmax, top-k and grouping in that GEMM's blocks
  // (RoutePrologue: the router's own top-k code, so the same ids, weights
  // and rows), which saves the one-wave top-k launch; the router launch
  // then writes the split logits only.
  if (decode_router) {
    ScopedTimer t(FMOE_TIMER_ROUTER, s, c.timers);
    const int nv = (E32 + 15) / 16;
    const int rnv = nv <= 1 ? 1 : nv <= 4 ? 4 : nv <= 8 ? 8 : 0;
    int v = 0;
    GroupedGemmArgs gr = g;
    RoutePrologue& rp = gr.rp;
    rp.part = at<float>(workspace, L.rpart);
    rp.n_split = router_decode_splits(H32);
    rp.k = k32;
    rp.normalize = c.normalize_weights != 0;
    rp.nv = rnv;
    rp.ids = ids;
    rp.weights = rw;
    rp.order = order;
    rp.offsets = offsets;
    rp.err_count = err;
    if (g_path.load(std::memory_order_relaxed) == FMOE_PATH_AUTO && T <= 4 && k32 * T <= 64 && rnv > 0 &&
        pick_path(g, &v) == FMOE_PATH_STREAM && gemm_stream_routed_ok(gr)) {
      int n_split = 0;
      FMOE_HIP(launch_router_split_logits(c.input, c.w_router, T, H32, E32, k32, act_dtype,
                                          at<float>(workspace, L.rpart), &n_split, s));
      if (n_split != rp.n_split) return fail(FMOE_ERR_HIP, "split logits: %d splits, %d expected", n_split, rp.n_split);
      g = gr;
    } else {
      FMOE_HIP(launch_router_decode(c.input, c.w_router, T, H32, E32, k32, c.normalize_weights != 0, act_dtype,
                                    at<float>(workspace, L.rpart), ids, rw, order, offsets, err, s));
    }
  } else {
    ScopedTimer t(FMOE_TIMER_ROUTER, s, c.timers);
    if (split_router)
      FMOE_HIP(launch_router_prefill(c.input, c.w_router, T, H32, E32, k32, c.normalize_weights != 0, act_dtype,
                                     at<float>(workspace, L.rpart), ids, rw, s));
    else
      FMOE_HIP(launch_router(c.input, c.w_router, T, H32, E32, k32, c.normalize_weights != 0, act_dtype, ids, rw,
                             s));
  }

  if (!decode_router) {
    // Tile schedules the permutation builds beside its scatter: those of the
    // 256-tile GEMMs that will run.
    TileTableReq reqs[kPermuteMaxTables];
    int n_req = 0;
    GroupedGemmArgs* dn = h_quant ? &dq : &d;
    for (GroupedGemmArgs* x : {&g, dn}) {
      if (!x->tile_table || !gemm_tiled256_table_request(*x, &reqs[n_req])) continue;
      int v = 0;
      const int path = pick_path(*x, &v);
      if ((path == FMOE_PATH_TILED || path == FMOE_PATH_TILED_LARGE) && v == TILED_256) {
        x->tile_table_ready = true;
        ++n_req;
      }
    }
    ScopedTimer t(FMOE_TIMER_PERMUTE, s, c.timers);
    FMOE_HIP(launch_permute(ids, n, static_cast<int>(n_expert), order, offsets, err,
                            at<int>(workspace, L.perm.scratch), s, reqs, n_req));
  }
  if (h_quant) {
    ScopedTimer t(FMOE_TIMER_QUANT, s, c.timers);
    // max |x| per token (that pass also clears the per-row max the gate/up
    // epilogue accumulates for h), then the token rows gathered into expert
    // order and quantised.
    FMOE_HIP(launch_row_absmax(c.input, T, static_cast<int>(n_embd), at<unsigned>(workspace, L.xmax),
                               at<unsigned>(workspace, L.hmax), n, s));
    FMOE_HIP(launch_quantize_rows_kb(c.input, order, n, T, static_cast<int>(n_embd), at<unsigned>(workspace, L.xmax),
                                     at<char>(workspace, L.xq), at<float>(workspace, L.xs), nullptr, s,
                                     L.x_plane ? at<char>(workspace, L.xq + L.x_plane) : nullptr));
  }
  if (gather_x) {
    ScopedTimer t(FMOE_TIMER_PERMUTE, s, c.timers);
    FMOE_HIP(launch_gather_rows_kb(c.input, order, n, T, static_cast<int>(n_embd), at<char>(workspace, L.xkb), s));
  }
  {
    ScopedTimer t(FMOE_TIMER_GATE_UP, s, c.timers);
    FMOE_TRY(run_grouped_gemm(g, s));
  }
  if (h_quant) {
    ScopedTimer t(FMOE_TIMER_QUANT, s, c.timers);
    FMOE_HIP(launch_quantize_rows_kb(h, nullptr, n, n, static_cast<int>(n_ff), at<unsigned>(workspace, L.hmax),
                                     at<char>(workspace, L.hq), at<float>(workspace, L.hs), nullptr, s,
                                     L.h_plane ? at<char>(workspace, L.hq + L.h_plane) : nullptr));
    d = dq;
  }

  // Decode batches of at most 16 assignments on the streaming kernel (the
  // automatic kernel choice): steps 9-11 in one launch.
  if (g_path.load(std::memory_order_relaxed) == FMOE_PATH_AUTO && n <= 16) {
    int vd = 0;
    if (pick_path(d, &vd) == FMOE_PATH_STREAM) {
      hipError_t e;
      {
        ScopedTimer t(FMOE_TIMER_DOWN, s, c.timers);
        e = launch_down_combine_small(d, c.residual, c.out, act_dtype, T, static_cast<int>(n_expert_used), s);
      }
      if (e == hipSuccess) {
        g_last_path = FMOE_PATH_STREAM;
        return ok();
      }
      if (e != hipErrorNotSupported) return fail(FMOE_ERR_HIP, "down + combine launch: %s", hipGetErrorString(e));
    }
  }

  // Steps 9-10: down projection, routing weight applied per assignment (mlir:158-177).
  int down_split = 1;
  {
    ScopedTimer t(FMOE_TIMER_DOWN, s, c.timers);
    FMOE_TRY(run_grouped_gemm(d, s, &down_split));
  }

  // Step 11: slot-ordered sum + transpose to [n_tokens, n_embd] (mlir:179-206),
  // plus the residual for the sub-layer.
  {
    ScopedTimer t(FMOE_TIMER_COMBINE, s, c.timers);
    FMOE_HIP(launch_combine(y, y_dtype, c.residual, c.out, act_dtype, T, static_cast<int>(n_expert_used),
                            static_cast<int>(n_embd), down_split, L.y_part_elems, s));
  }
  return ok();
}

// ------------------------------------------------------------ attention half
// Shapes shared by the attention entry points.
struct AttnShape {
  int64_t B, n_head, n_head_kv, n_embd, n_embd_kv, D;
};

int validate_attn_shape(const AttnShape& a, int act_dtype, int w_dtype) {
  if (!act_dtype_ok(act_dtype)) return fail(FMOE_ERR_DTYPE, "activation dtype %d", act_dtype);
  if (!w_dtype_ok(w_dtype)) return fail(FMOE_ERR_DTYPE, "weight dtype %d", w_dtype);
  if (act_dtype == FMOE_F32 && w_dtype != FMOE_F32) return fail(FMOE_ERR_DTYPE, "f32 activations need f32 weights");
  FMOE_TRY(check_dims("batch", a.B, 0, 65535));
  FMOE_TRY(check_dims("n_head", a.n_head, 1, 65535));
  FMOE_TRY(check_dims("n_head_kv", a.n_head_kv, 1, a.n_head));
  FMOE_TRY(check_dims("n_embd", a.n_embd, 1, kMaxDim));
  FMOE_TRY(check_dims("n_embd_kv", a.n_embd_kv, 1, kMaxDim));
  if (a.n_head % a.n_head_kv) return fail(FMOE_ERR_SHAPE, "n_head %% n_head_kv != 0");
  if (a.n_embd % a.n_head || a.n_embd_kv % a.n_head_kv || a.n_embd / a.n_head != a.n_embd_kv / a.n_head_kv)
    return fail(FMOE_ERR_SHAPE, "head_dim must be n_embd / n_head = n_embd_kv / n_head_kv");
  if (!attn_decode_supported(static_cast<int>(a.D), static_cast<int>(a.n_head / a.n_head_kv)))
    return fail(FMOE_ERR_SHAPE, "head_dim %lld with %lld query heads per KV head is not supported "
                "(head_dim 16/32/64/128, group 1/2/4/8)", static_cast<long long>(a.D),
                static_cast<long long>(a.n_head / a.n_head_kv));
  if (a.n_embd + 2 * a.n_embd_kv > kMaxDim) return fail(FMOE_ERR_SHAPE, "n_embd + 2 n_embd_kv too large");
  return FMOE_OK;
}

// K splits a decode projection may use (fp32 partials in the workspace).
constexpr int kLinearMaxSplit = 8;

struct AttnLayout {
  size_t order, offsets, tables, lens, qkv, q_rot, k_new, v_new, part, attn, y, total;
};

AttnLayout attn_layout(const AttnShape& a, int64_t max_ctx, int act) {
  AttnLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at_ = off;
    off += align_up(bytes);
    return at_;
  };
  const size_t ab = dtype_bytes(act);
  L.order = take(static_cast<size_t>(a.B) * 4);
  L.offsets = take(2 * 4);
  L.tables = take(static_cast<size_t>(a.B) * 4);
  L.lens = take(static_cast<size_t>(a.B) * 4);
  L.qkv = take(static_cast<size_t>(a.B) * (a.n_embd + 2 * a.n_embd_kv) * 4 * kLinearMaxSplit);
  L.q_rot = take(static_cast<size_t>(a.B) * a.n_embd * 4);
  L.k_new = take(static_cast<size_t>(a.B) * a.n_embd_kv * ab);
  L.v_new = take(static_cast<size_t>(a.B) * a.n_embd_kv * ab);
  L.part = take(static_cast<size_t>(a.B) * a.n_head * attn_decode_splits(static_cast<int>(max_ctx)) * (a.D + 2) * 4);
  L.attn = take(static_cast<size_t>(a.B) * a.n_embd * ab);
  L.y = take(static_cast<size_t>(a.B) * a.n_embd * 4 * kLinearMaxSplit);
  L.total = off;
  return L;
}

// Rows up to which a one-expert projection streams its weight (K split over
// fp32 partials); above it, the 256-row tile kernel with K split.  Measured
// on the decode attention's projections (n_embd 4096): at 64 rows the tile
// kernel takes the Q/K/V product from 39 to 32 us, at 128 rows from 88 (the
// unsplit tile kernel) to 38 us and the output projection from 84 to 31 us;
// at 32 rows streaming is ahead (Q/K/V 27 against 29 us).  The fused
// epilogues below stream up to 64 rows (the output projection with its bias
// and residual at 64 rows: 24.7 us, level with the split product + launch).
constexpr int kLinearStreamRows = 32;

// out[B, N] fp32 = x[B, K] @ W for a one-expert packed weight [N, K].  The
// streaming kernel reads the B rows in order with no grouping arrays and
// splits K so that the few column tiles of one weight still fill the GPU:
// *nsplit partial sums, B * N floats apart, to be added in order.  The other
// paths get the identity grouping written into order [B] / offsets [2].
// With `pe` the streaming kernel applies that epilogue itself (no K split,
// `out` unused) where it supports it, and *fused reports whether it did.
int run_linear(const void* x, int64_t K, const void* packed, const float* scales, int w_dtype, int64_t N, float* out,
               int B, int act, int* order, int* offsets, hipStream_t s, int* nsplit,
               const ProjEpilogue* pe = nullptr, bool* fused = nullptr) {
  const int out_dtype = FMOE_F32;
  *nsplit = 1;
  if (fused) *fused = false;
  GroupedGemmArgs g;
  g.a = x;
  g.lda = K;
  g.a_mode = A_DIRECT;
  g.order = nullptr;
  g.offsets = nullptr;
  g.n_tokens = B;
  g.n_assign = B;
  g.n_expert = 1;
  g.w0 = packed;
  g.s0 = w_dtype == FMOE_F8E4M3FN ? scales : nullptr;
  g.N = N;
  g.K = K;
  g.out = out;
  g.ldo = N;
  g.epi = EPI_SCATTER;
  g.act_dtype = act;
  g.w_dtype = w_dtype;
  g.w_format = packed_format(N, K, w_dtype);
  g.out_dtype = out_dtype;
  g.max_rows_per_expert = B;
  // Decode batches read each weight once in the streaming kernel (see
  // kLinearStreamRows), with up to ~2048 blocks and at least 4 input steps
  // per wave.
  if (g_path.load(std::memory_order_relaxed) == FMOE_PATH_AUTO && B <= 64 && pe && fused) {
    GroupedGemmArgs f = g;
    f.epi = pe->kind;
    f.pe = *pe;
    f.out = pe->kind == EPI_LINEAR ? pe->out : nullptr;
    f.out_dtype = FMOE_BF16;
    if (gemm_stream_supported(f)) {
      FMOE_HIP(launch_gemm_stream(f, s));
      g_last_path = FMOE_PATH_STREAM;
      *fused = true;
      return FMOE_OK;
    }
  }
  if (g_path.load(std::memory_order_relaxed) == FMOE_PATH_AUTO && B <= kLinearStreamRows && gemm_stream_supported(g)) {
    // Split K so that each wave streams one full trip of 8 steps (K / 32 /
    // (4 waves * 8)) while the grid has fewer than ~2048 blocks.
    const int64_t tiles = (N + 15) / 16;
    const int64_t steps = K / 32;
    int64_t ks = std::min<int64_t>(steps / 32, (2048 + tiles - 1) / tiles);
    ks = std::max<int64_t>(1, std::min<int64_t>(ks, kLinearMaxSplit));
    g.ksplit = static_cast<int>(ks);
    g.split_stride = static_cast<int64_t>(B) * N;
    FMOE_HIP(launch_gemm_stream(g, s));
    g_last_path = FMOE_PATH_STREAM;
    *nsplit = g.ksplit;
    return FMOE_OK;
  }
  g.order = order;
  g.offsets = offsets;
  FMOE_HIP(launch_iota(order, B, offsets, 0, B, s));
  // Larger batches: the 256-row tile kernel, K split so that the few column
  // tiles of one weight still give the GPU about 256 blocks.
  if (g_path.load(std::memory_order_relaxed) == FMOE_PATH_AUTO) {
    GroupedGemmArgs t = g;
    t.split_stride = static_cast<int64_t>(B) * N;
    const int64_t tiles = static_cast<int64_t>(max_row_tiles(B, 1, 256)) * ((N + 255) / 256);
    int ks = 1;
    while (ks * 2 <= kLinearMaxSplit && tiles * ks * 2 <= 256) ks *= 2;
    t.ksplit = ks;
    while (t.ksplit > 1 && !gemm_tiled256_supported(t)) t.ksplit /= 2;
    if (t.ksplit > 1) {
      FMOE_HIP(launch_gemm_tiled(t, s, TILED_256));
      g_last_path = FMOE_PATH_TILED_LARGE;
      *nsplit = t.ksplit;
      return FMOE_OK;
    }
  }
  return run_grouped_gemm(g, s);
}

struct AttnWeights {
  const void* wqkv;
  const float* wqkv_scales;
  const void* wo;
  const float* wo_scales;
  int w_dtype;
  const float *bq, *bk, *bv, *bo;
  int use_bias;
  float freq_base, freq_scale;
};

// Projections, RoPE, attention over the pools and the output projection
// (attention_block_decode.mlir:96-233).  k_new / v_new: [B, n_embd_kv] in
// act dtype (RoPE applied to k_new).
int run_attention(const AttnShape& a, const AttnWeights& w, const void* input, const int64_t* positions,
                  const void* k_pool, const void* v_pool, int64_t n_blocks, int block_size, const int* tables,
                  int max_blocks, const int* lens, int max_ctx, int act, void* out, void* k_new, void* v_new,
                  void* workspace, const AttnLayout& L, hipStream_t s, const void* residual = nullptr,
                  const KvScatterDecode* scatter = nullptr) {
  const int B = static_cast<int>(a.B);
  const int nq = static_cast<int>(a.n_embd), nkv = static_cast<int>(a.n_embd_kv);
  int* order = at<int>(workspace, L.order);
  int* offsets = at<int>(workspace, L.offsets);
  float* qkv = at<float>(workspace, L.qkv);
  float* q_rot = at<float>(workspace, L.q_rot);
  const bool bias = w.use_bias != 0;
  {
    ScopedTimer t(FMOE_TIMER_QKV, s);
    // bias + RoPE in the GEMM's epilogue where the streaming kernel takes
    // it, else over the fp32 (K-split) result.  Fused only up to 16 rows:
    // the epilogue's double-precision angles run on one wave per block, and
    // at 64 rows the separate RoPE launch is faster (Q/K/V phase 38.6
    // against 44.5 us fused at 64 x 1024 positions).  At 16 x 4096 the
    // fused step is 1.3 us shorter, at 1 x 512 3.5 us (43.0 -> 39.5 us).
    ProjEpilogue pe;
    pe.kind = EPI_QKV_ROPE;
    pe.bias = bias ? w.bq : nullptr;
    pe.bias_k = bias ? w.bk : nullptr;
    pe.bias_v = bias ? w.bv : nullptr;
    pe.positions = positions;
    pe.nq = nq;
    pe.nkv = nkv;
    pe.head_dim = static_cast<int>(a.D);
    pe.freq_base = w.freq_base;
    pe.freq_scale = w.freq_scale;
    pe.q_out = q_rot;
    pe.k_out = k_new;
    pe.v_out = v_new;
    int ns = 1;
    bool fused = false;
    FMOE_TRY(run_linear(input, a.n_embd, w.wqkv, w.wqkv_scales, w.w_dtype, nq + 2 * nkv, qkv, B, act, order,
                        offsets, s, &ns, act == FMOE_BF16 && B <= 16 ? &pe : nullptr, &fused));
    if (!fused)
      FMOE_HIP(launch_qkv_rope(qkv, ns, static_cast<int64_t>(B) * (nq + 2 * nkv), bias ? w.bq : nullptr,
                               bias ? w.bk : nullptr, bias ? w.bv : nullptr, positions, B, nq, nkv,
                               static_cast<int>(a.D), w.freq_base, w.freq_scale, q_rot, k_new, v_new, act, s));
  }
  void* attn = at<char>(workspace, L.attn);
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(a.D)));
  {
    ScopedTimer t(FMOE_TIMER_ATTENTION, s);
    FMOE_HIP(launch_attn_decode(q_rot, k_pool, v_pool, n_blocks, block_size, tables, max_blocks, lens, max_ctx, k_new,
                                v_new, B, static_cast<int>(a.n_head), static_cast<int>(a.n_head_kv),
                                static_cast<int>(a.D), act, scale, at<float>(workspace, L.part), attn, s, scatter));
  }
  float* y = at<float>(workspace, L.y);
  {
    ScopedTimer t(FMOE_TIMER_OUT_PROJ, s);
    ProjEpilogue pe;
    pe.kind = EPI_LINEAR;
    pe.bias = bias ? w.bo : nullptr;
    pe.residual = residual;
    pe.out = out;
    int ns = 1;
    bool fused = false;
    FMOE_TRY(run_linear(attn, a.n_embd, w.wo, w.wo_scales, w.w_dtype, nq, y, B, act, order, offsets, s, &ns,
                        act == FMOE_BF16 ? &pe : nullptr, &fused));
    if (!fused)
      FMOE_HIP(launch_bias_cast(y, ns, static_cast<int64_t>(B) * nq, bias ? w.bo : nullptr, residual, out, B, nq,
                                act, s));
  }
  return FMOE_OK;
}

int check_attn_weights(const AttnWeights& w) {
  if (!w.wqkv || !w.wo) return fail(FMOE_ERR_INVALID_ARGUMENT, "null weight");
  if (w.w_dtype == FMOE_F8E4M3FN && (!w.wqkv_scales || !w.wo_scales))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "fp8 weights need scales");
  if (w.use_bias != 0 && w.use_bias != 1) return fail(FMOE_ERR_INVALID_ARGUMENT, "use_bias must be 0 or 1");
  if (w.use_bias && (!w.bq || !w.bk || !w.bv || !w.bo)) return fail(FMOE_ERR_INVALID_ARGUMENT, "null bias");
  return FMOE_OK;
}

// Pools are addressed by a 32-bit row index (block * block_size + row).
int check_pool(int64_t n_blocks, int64_t block_size) {
  FMOE_TRY(check_dims("n_blocks", n_blocks, 1, kMaxDim));
  FMOE_TRY(check_dims("block_size", block_size, 1, kMaxDim));
  if (n_blocks * block_size > kMaxDim) return fail(FMOE_ERR_SHAPE, "n_blocks * block_size exceeds 2^31-1");
  return FMOE_OK;
}

}  // namespace

extern "C" {

const char* fmoe_last_error(void) { return g_err; }

int fmoe_abi_version(void) { return FMOE_ABI_VERSION; }

int fmoe_device_check(int* device, char* arch, size_t arch_len) {
  FMOE_TRY(ensure_device(device, arch, arch_len));
  return ok();
}

int fmoe_set_gemm_path(int path) {
  if (path < FMOE_PATH_AUTO || path > FMOE_PATH_TILED_LARGE)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "unknown gemm path %d", path);
  g_path.store(path);
  return ok();
}

int fmoe_get_gemm_path(void) { return g_path.load(); }

int fmoe_quantize_rows_e4m3(const void* src, int64_t n_rows, int64_t n_cols, void* dst_hi, void* dst_lo,
                            float* dst_scale, void* stream) {
  FMOE_TRY(check_dims("n_rows", n_rows, 0, kMaxDim));
  FMOE_TRY(check_dims("n_cols", n_cols, 64, 16384));
  if (n_cols % 64) return fail(FMOE_ERR_SHAPE, "n_cols=%lld is not a multiple of 64", static_cast<long long>(n_cols));
  if (n_rows == 0) return ok();
  if (!src || !dst_hi || !dst_scale) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_quantize_rows_kb(src, nullptr, static_cast<int>(n_rows), static_cast<int>(n_rows),
                                   static_cast<int>(n_cols), nullptr, dst_hi, dst_scale, nullptr,
                                   static_cast<hipStream_t>(stream), dst_lo));
  return ok();
}

int fmoe_last_gemm_path(void) { return g_last_path; }

int fmoe_timing_enable(int on) {
  g_timing.store(on != 0);
  return ok();
}

int fmoe_timing_read(double* ms_out, int64_t* regions_out, int n) {
  std::lock_guard<std::mutex> lk(g_t_mu);
  for (const PendingTiming& p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      g_t_ms[p.timer] += ms;
      g_t_calls[p.timer] += 1;
    }
    g_event_pool.push_back(p.start);
    g_event_pool.push_back(p.stop);
  }
  g_pending.clear();
  for (int i = 0; i < n && i < FMOE_TIMER_COUNT; ++i) {
    if (ms_out) ms_out[i] = g_t_ms[i];
    if (regions_out) regions_out[i] = g_t_calls[i];
  }
  for (int i = 0; i < FMOE_TIMER_COUNT; ++i) {
    g_t_ms[i] = 0;
    g_t_calls[i] = 0;
  }
  return ok();
}

int fmoe_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  if (!act_dtype_ok(dtype)) return fail(FMOE_ERR_DTYPE, "swiglu dtype %d not F32/BF16", dtype);
  FMOE_TRY(check_dims("n", n, 0, (1ll << 62)));
  if (n == 0) return ok();
  if (!gate || !up || !out) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (!aligned_for(gate, dtype) || !aligned_for(up, dtype) || !aligned_for(out, dtype))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_swiglu(gate, up, out, n, dtype, static_cast<hipStream_t>(stream)));
  return ok();
}

int fmoe_router(const void* input, const void* w_router, int64_t n_tokens, int64_t n_embd,
                int64_t n_expert, int64_t n_expert_used, int normalize_weights, int dtype,
                int32_t* ids_out, float* weights_out, void* stream) {
  if (!act_dtype_ok(dtype)) return fail(FMOE_ERR_DTYPE, "router dtype %d not F32/BF16", dtype);
  FMOE_TRY(validate_router(n_tokens, n_embd, n_expert, n_expert_used));
  if (normalize_weights != 0 && normalize_weights != 1)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "normalize_weights must be 0 or 1");
  if (n_tokens == 0) return ok();
  if (!input || !w_router || !ids_out || !weights_out)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_router(input, w_router, static_cast<int>(n_tokens), static_cast<int>(n_embd),
                         static_cast<int>(n_expert), static_cast<int>(n_expert_used),
                         normalize_weights != 0, dtype, ids_out, weights_out,
                         static_cast<hipStream_t>(stream)));
  return ok();
}

size_t fmoe_permute_workspace_bytes(int64_t n_expert_used, int64_t n_tokens, int64_t n_expert) {
  // error word, then the chunk histograms of a large batch
  if (n_expert_used < 1 || n_tokens < 0 || n_expert < 1 || n_expert > 512 || n_expert_used * n_tokens > kMaxDim)
    return align_up(16);
  return align_up(16) + align_up(permute_scratch_bytes(static_cast<int>(n_expert_used * n_tokens),
                                                       static_cast<int>(n_expert)));
}

int fmoe_permute(const int32_t* ids, int64_t n_expert_used, int64_t n_tokens, int64_t n_expert,
                 int32_t* order_out, int32_t* offsets_out, void* workspace,
                 size_t workspace_bytes, void* stream) {
  FMOE_TRY(check_dims("n_tokens", n_tokens, 0, kMaxDim));
  FMOE_TRY(check_dims("n_expert", n_expert, 1, 512));
  FMOE_TRY(check_dims("n_expert_used", n_expert_used, 1, kMaxDim));
  if (n_expert_used * n_tokens > kMaxDim)
    return fail(FMOE_ERR_SHAPE, "n_expert_used * n_tokens exceeds 2^31-1");
  if (!offsets_out || !workspace) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (workspace_bytes < fmoe_permute_workspace_bytes(n_expert_used, n_tokens, n_expert))
    return fail(FMOE_ERR_WORKSPACE, "workspace too small");
  if (n_tokens > 0 && (!ids || !order_out)) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_permute(ids, static_cast<int>(n_expert_used * n_tokens),
                          static_cast<int>(n_expert), order_out, offsets_out,
                          static_cast<int*>(workspace), at<int>(workspace, align_up(16)),
                          static_cast<hipStream_t>(stream)));
  return ok();
}

int fmoe_workspace_error_count(const void* workspace, void* stream, int64_t* count_out) {
  if (!workspace || !count_out) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  FMOE_TRY(ensure_device());
  int v = 0;
  FMOE_HIP(hipMemcpyAsync(&v, workspace, sizeof(int), hipMemcpyDeviceToHost,
                          static_cast<hipStream_t>(stream)));
  FMOE_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  *count_out = v;
  return ok();
}

size_t fmoe_packed_weight_bytes(int64_t n_out, int64_t n_in, int64_t n_expert, int dtype) {
  if (n_out < 0 || n_in < 0 || n_expert < 0 || !w_dtype_ok(dtype)) return 0;
  // + a tail the tiled kernels may read (never use) past the last expert
  return static_cast<size_t>(n_out) * n_in * n_expert * dtype_bytes(dtype) +
         static_cast<size_t>(kPackedTailRows) * n_in * 2;
}

int fmoe_pack_expert_weights(const void* src, int src_dtype, const float* src_scales,
                             int64_t n_out, int64_t n_in, int64_t n_expert, int dst_dtype,
                             void* dst, float* dst_scales, void* stream) {
  if (!w_dtype_ok(src_dtype) || !w_dtype_ok(dst_dtype))
    return fail(FMOE_ERR_DTYPE, "pack dtypes %d -> %d", src_dtype, dst_dtype);
  if (src_dtype == FMOE_F8E4M3FN && dst_dtype != FMOE_F8E4M3FN)
    return fail(FMOE_ERR_DTYPE, "fp8 weights can only be packed as fp8");
  FMOE_TRY(check_dims("n_out", n_out, 0, kMaxDim));
  FMOE_TRY(check_dims("n_in", n_in, 0, kMaxDim));
  FMOE_TRY(check_dims("n_expert", n_expert, 1, 1024));
  if (n_out == 0 || n_in == 0) return ok();
  if (!src || !dst) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (src_dtype == FMOE_F8E4M3FN && !src_scales)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "fp8 source needs src_scales");
  if (dst_dtype == FMOE_F8E4M3FN && !dst_scales)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "fp8 destination needs dst_scales");
  if (!aligned_for(src, src_dtype) || !aligned_for(dst, dst_dtype))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_pack(src, src_dtype, src_scales, static_cast<int>(n_out), static_cast<int>(n_in),
                       static_cast<int>(n_expert), dst_dtype, dst, dst_scales,
                       static_cast<hipStream_t>(stream)));
  return ok();
}

size_t fmoe_mul_mat_id_workspace_bytes(int64_t n_out, int64_t n_in, int64_t n_expert,
                                       int64_t n_expert_used, int64_t n_tokens, int act_dtype) {
  if (!act_dtype_ok(act_dtype) || n_out < 0 || n_in < 0 || n_expert < 1 || n_expert_used < 0 ||
      n_tokens < 0)
    return 0;
  return mmid_layout(n_out, n_in, n_expert, n_expert_used, n_tokens, act_dtype).total;
}

int fmoe_mul_mat_id(const void* packed_w, const float* w_scales, int w_dtype, const void* input,
                    const int32_t* ids, void* out, int64_t n_out, int64_t n_in, int64_t n_expert,
                    int64_t n_expert_used, int64_t n_tokens, int act_dtype, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (!act_dtype_ok(act_dtype)) return fail(FMOE_ERR_DTYPE, "activation dtype %d", act_dtype);
  if (!w_dtype_ok(w_dtype)) return fail(FMOE_ERR_DTYPE, "weight dtype %d", w_dtype);
  if (act_dtype == FMOE_F32 && w_dtype != FMOE_F32)
    return fail(FMOE_ERR_DTYPE, "f32 activations need f32 weights");
  FMOE_TRY(check_dims("n_out", n_out, 0, kMaxDim));
  FMOE_TRY(check_dims("n_in", n_in, 0, kMaxDim));
  FMOE_TRY(check_dims("n_expert", n_expert, 1, 512));
  FMOE_TRY(check_dims("n_expert_used", n_expert_used, 1, kMaxDim));
  FMOE_TRY(check_dims("n_tokens", n_tokens, 0, kMaxDim));
  const int64_t n = n_expert_used * n_tokens;
  if (n > kMaxDim) return fail(FMOE_ERR_SHAPE, "n_expert_used * n_tokens exceeds 2^31-1");
  if (n == 0 || n_out == 0) return ok();
  if (!packed_w || !input || !ids || !out || !workspace)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (w_dtype == FMOE_F8E4M3FN && !w_scales)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "fp8 weights need scales");
  const MmidLayout L = mmid_layout(n_out, n_in, n_expert, n_expert_used, n_tokens, act_dtype);
  if (workspace_bytes < L.total)
    return fail(FMOE_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", workspace_bytes, L.total);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "workspace must be %zu-byte aligned", kAlign);
  if (!aligned_for(input, act_dtype) || !aligned_for(out, act_dtype))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  FMOE_TRY(ensure_device());
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* err = at<int>(workspace, L.perm.err);
  int* order = at<int>(workspace, L.perm.order);
  int* offsets = at<int>(workspace, L.perm.offsets);
  void* x = at<char>(workspace, L.x);
  void* y = at<char>(workspace, L.y);
  // input [n_in, k*T] -> x [k*T, n_in]: row f = s*T + t (mul_mat_id.mlir:63-90)
  if (n_in > 0) FMOE_HIP(launch_transpose(input, x, n_in, n, act_dtype, s));
  FMOE_HIP(launch_permute(ids, static_cast<int>(n), static_cast<int>(n_expert), order, offsets, err,
                          at<int>(workspace, L.perm.scratch), s));
  GroupedGemmArgs g;
  g.a = x;
  g.lda = n_in;
  g.a_mode = A_GATHER_FLAT;
  g.order = order;
  g.offsets = offsets;
  g.n_tokens = static_cast<int>(n_tokens);
  g.n_assign = static_cast<int>(n);
  g.n_expert = static_cast<int>(n_expert);
  g.w0 = packed_w;
  g.s0 = w_dtype == FMOE_F8E4M3FN ? w_scales : nullptr;
  g.N = n_out;
  g.K = n_in;
  g.out = y;
  g.ldo = n_out;
  g.epi = EPI_SCATTER;
  g.act_dtype = act_dtype;
  g.w_dtype = w_dtype;
  g.w_format = packed_format(n_out, n_in, w_dtype);
  g.out_dtype = act_dtype;
  {
    ScopedTimer t(FMOE_TIMER_MUL_MAT_ID, s);
    FMOE_TRY(run_grouped_gemm(g, s));
  }
  FMOE_HIP(launch_zero_invalid_rows(ids, static_cast<int>(n), static_cast<int>(n_expert), y,
                                    act_dtype, n_out, s));
  // y [k*T, n_out] -> out [n_out, k*T] (mul_mat_id.mlir:96-117)
  FMOE_HIP(launch_transpose(y, out, n, n_out, act_dtype, s));
  return ok();
}

size_t fmoe_moe_ffn_block_workspace_bytes(int64_t n_tokens, int64_t n_expert,
                                          int64_t n_expert_used, int64_t n_embd, int64_t n_ff,
                                          int act_dtype, int w_dtype) {
  if (!act_dtype_ok(act_dtype) || !block_w_dtype_ok(w_dtype) || n_tokens < 0 || n_expert < 1 ||
      n_expert_used < 1 || n_embd < 1 || n_ff < 0)
    return 0;
  return block_layout(n_tokens, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype).total;
}

int fmoe_moe_ffn_block(const void* input, const void* w_router, const void* packed_up,
                       const void* packed_gate, const void* packed_down, const float* up_scales,
                       const float* gate_scales, const float* down_scales, int w_dtype, void* out,
                       int64_t n_tokens, int64_t n_expert, int64_t n_expert_used, int64_t n_embd,
                       int64_t n_ff, int normalize_weights, int act_dtype, void* workspace,
                       size_t workspace_bytes, void* stream) {
  const BlockCall c{input,     w_router,   packed_up,     packed_gate, packed_down,       up_scales,
                    gate_scales, down_scales, w_dtype,    out,         nullptr,           n_tokens,
                    n_expert,  n_expert_used, n_embd,     n_ff,        normalize_weights, act_dtype,
                    workspace, workspace_bytes, stream};
  FMOE_TRY(validate_block(c));
  if (n_tokens == 0) return ok();
  const BlockLayout L = block_layout(n_tokens, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype);
  FMOE_TRY(check_workspace(workspace, workspace_bytes, L.total));
  FMOE_TRY(ensure_device());
  return run_block(c, L);
}

int fmoe_moe_ffn_block_noalloc(const void* input, const void* w_router, const void* packed_up,
                               const void* packed_gate, const void* packed_down, const float* up_scales,
                               const float* gate_scales, const float* down_scales, int w_dtype, void* out,
                               int64_t n_tokens, int64_t n_expert, int64_t n_expert_used, int64_t n_embd,
                               int64_t n_ff, int normalize_weights, int act_dtype, void* stream) {
  BlockCall c{input,     w_router,   packed_up,     packed_gate, packed_down,       up_scales,
              gate_scales, down_scales, w_dtype,    out,         nullptr,           n_tokens,
              n_expert,  n_expert_used, n_embd,     n_ff,        normalize_weights, act_dtype,
              nullptr,   0,          stream};
  c.timers = false;
  FMOE_TRY(validate_block(c));
  if (n_tokens == 0) return ok();
  const BlockLayout L = block_layout(n_tokens, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype);
  if (L.total > FMOE_NOALLOC_SCRATCH_BYTES)
    return fail(FMOE_ERR_WORKSPACE,
                "fmoe_moe_ffn_block_noalloc: %lld tokens need %zu bytes of scratch, above its fixed %zu bytes "
                "(FMOE_NOALLOC_SCRATCH_BYTES); use fmoe_moe_ffn_block with a workspace",
                static_cast<long long>(n_tokens), L.total, static_cast<size_t>(FMOE_NOALLOC_SCRATCH_BYTES));
  int dev = 0;
  FMOE_TRY(ensure_device(&dev));
  // The scratch array's device address on this device (hipGetSymbolAddress
  // on first use, then cached); never the array itself.
  void* scratch = nullptr;
  FMOE_HIP(noalloc_scratch(dev, &scratch));
  c.workspace = scratch;
  c.workspace_bytes = FMOE_NOALLOC_SCRATCH_BYTES;
  return run_block(c, L);
}

int fmoe_rms_norm(const void* input, const void* weight, float eps, void* out, int64_t n_rows,
                  int64_t n_embd, int dtype, void* stream) {
  if (!act_dtype_ok(dtype)) return fail(FMOE_ERR_DTYPE, "dtype %d", dtype);
  FMOE_TRY(check_dims("n_rows", n_rows, 0, kMaxDim));
  FMOE_TRY(check_dims("n_embd", n_embd, 1, kMaxDim));
  if (n_rows == 0) return ok();
  if (!input || !weight || !out) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (!aligned_for(input, dtype) || !aligned_for(weight, dtype) || !aligned_for(out, dtype))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_rms_norm(input, weight, eps, out, n_rows, static_cast<int>(n_embd), dtype,
                           static_cast<hipStream_t>(stream)));
  return ok();
}

size_t fmoe_moe_ffn_sublayer_workspace_bytes(int64_t n_tokens, int64_t n_expert, int64_t n_expert_used,
                                             int64_t n_embd, int64_t n_ff, int act_dtype, int w_dtype) {
  if (!act_dtype_ok(act_dtype) || !block_w_dtype_ok(w_dtype) || n_tokens < 0 || n_expert < 1 ||
      n_expert_used < 1 || n_embd < 1 || n_ff < 0)
    return 0;
  return sublayer_layout(n_tokens, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype).total;
}

int fmoe_moe_ffn_sublayer(const void* residual, const void* ffn_norm_w, float rms_eps, const void* w_router,
                          const void* packed_up, const void* packed_gate, const void* packed_down,
                          const float* up_scales, const float* gate_scales, const float* down_scales,
                          int w_dtype, void* out, int64_t n_tokens, int64_t n_expert, int64_t n_expert_used,
                          int64_t n_embd, int64_t n_ff, int normalize_weights, int act_dtype, void* workspace,
                          size_t workspace_bytes, void* stream) {
  BlockCall c{residual,  w_router,   packed_up,     packed_gate, packed_down,       up_scales,
              gate_scales, down_scales, w_dtype,    out,         residual,          n_tokens,
              n_expert,  n_expert_used, n_embd,     n_ff,        normalize_weights, act_dtype,
              workspace, workspace_bytes, stream};
  FMOE_TRY(validate_block(c));
  if (n_tokens == 0) return ok();
  if (!ffn_norm_w) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (!aligned_for(ffn_norm_w, act_dtype)) return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  const SublayerLayout SL = sublayer_layout(n_tokens, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype);
  FMOE_TRY(check_workspace(workspace, workspace_bytes, SL.total));
  FMOE_TRY(ensure_device());
  hipStream_t s = static_cast<hipStream_t>(stream);
  // ffn_norm (transformer_layer_moe_prefill.mlir:211-213): the normalised
  // rows feed the router and the gate/up GEMM; the residual goes to combine.
  void* xn = at<char>(workspace, SL.xn);
  {
    ScopedTimer t(FMOE_TIMER_NORM, s);
    FMOE_HIP(launch_rms_norm(residual, ffn_norm_w, rms_eps, xn, n_tokens, static_cast<int>(n_embd), act_dtype,
                             s));
  }
  c.input = xn;
  return run_block(c, SL.block);
}

int fmoe_moe_ffn_block_routing(void* workspace, int64_t n_tokens, int64_t n_expert,
                               int64_t n_expert_used, int64_t n_embd, int64_t n_ff, int act_dtype,
                               int w_dtype, int32_t** ids, float** weights, int32_t** order,
                               int32_t** offsets) {
  if (!workspace) return fail(FMOE_ERR_INVALID_ARGUMENT, "null workspace");
  if (!act_dtype_ok(act_dtype) || !block_w_dtype_ok(w_dtype)) return fail(FMOE_ERR_DTYPE, "dtype");
  const BlockLayout L = block_layout(n_tokens, n_expert, n_expert_used, n_embd, n_ff, act_dtype, w_dtype);
  if (ids) *ids = at<int32_t>(workspace, L.ids);
  if (weights) *weights = at<float>(workspace, L.weights);
  if (order) *order = at<int32_t>(workspace, L.perm.order);
  if (offsets) *offsets = at<int32_t>(workspace, L.perm.offsets);
  return ok();
}

// ------------------------------------------------------------ paged KV cache
static int kv_common(const void* cache, int dtype, int64_t n_blocks, int64_t block_size, int64_t n_head_kv,
                     int64_t head_dim, int* row_bytes) {
  if (!act_dtype_ok(dtype)) return fail(FMOE_ERR_DTYPE, "cache dtype %d", dtype);
  FMOE_TRY(check_dims("n_blocks", n_blocks, 1, kMaxDim));
  FMOE_TRY(check_dims("block_size", block_size, 1, kMaxDim));
  FMOE_TRY(check_dims("n_head_kv", n_head_kv, 1, 65535));
  FMOE_TRY(check_dims("head_dim", head_dim, 2, 65535));
  if (head_dim % 2) return fail(FMOE_ERR_SHAPE, "head_dim must be even");
  const int64_t rb = n_head_kv * head_dim * dtype_bytes(dtype);
  if (rb > (1 << 30)) return fail(FMOE_ERR_SHAPE, "row too large");
  if (!cache) return fail(FMOE_ERR_INVALID_ARGUMENT, "null cache");
  if (reinterpret_cast<uintptr_t>(cache) % 4) return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned cache");
  *row_bytes = static_cast<int>(rb);
  return FMOE_OK;
}

int fmoe_kvcache_gather(const void* cache, int dtype, int64_t n_blocks, int64_t block_size, int64_t n_head_kv,
                        int64_t head_dim, int64_t layer, const int32_t* block_tables, const int32_t* context_lens,
                        int64_t n_layers, int64_t batch, int64_t max_blocks_per_seq, int64_t max_context_len,
                        void* out, void* stream) {
  int rb = 0;
  FMOE_TRY(kv_common(cache, dtype, n_blocks, block_size, n_head_kv, head_dim, &rb));
  FMOE_TRY(check_dims("n_layers", n_layers, 1, kMaxDim));
  FMOE_TRY(check_dims("layer", layer, 0, n_layers - 1));
  FMOE_TRY(check_dims("batch", batch, 0, 65535));
  FMOE_TRY(check_dims("max_blocks_per_seq", max_blocks_per_seq, 1, kMaxDim));
  FMOE_TRY(check_dims("max_context_len", max_context_len, 0, kMaxDim));
  if (batch == 0 || max_context_len == 0) return ok();
  if (!block_tables || !context_lens || !out) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (reinterpret_cast<uintptr_t>(out) % 4) return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned out");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_kv_gather(cache, n_blocks, static_cast<int>(block_size), rb,
                            block_tables + layer * batch * max_blocks_per_seq, static_cast<int>(max_blocks_per_seq),
                            context_lens + layer * batch, static_cast<int>(max_context_len), static_cast<int>(batch),
                            out, static_cast<hipStream_t>(stream)));
  return ok();
}

int fmoe_kvcache_scatter_decode(void* cache, int dtype, int64_t n_blocks, int64_t block_size, int64_t n_head_kv,
                                int64_t head_dim, const void* new_vals, const int32_t* block_indices,
                                const int32_t* pos_in_blocks, int64_t batch, void* stream) {
  int rb = 0;
  FMOE_TRY(kv_common(cache, dtype, n_blocks, block_size, n_head_kv, head_dim, &rb));
  FMOE_TRY(check_dims("batch", batch, 0, kMaxDim));
  if (batch == 0) return ok();
  if (!new_vals || !block_indices || !pos_in_blocks) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (reinterpret_cast<uintptr_t>(new_vals) % 4) return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned new_vals");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_kv_scatter_decode(cache, n_blocks, static_cast<int>(block_size), rb, new_vals, block_indices,
                                    pos_in_blocks, static_cast<int>(batch), static_cast<hipStream_t>(stream)));
  return ok();
}

int fmoe_kvcache_scatter_prefill(void* cache, int dtype, int64_t n_blocks, int64_t block_size, int64_t n_head_kv,
                                 int64_t head_dim, int64_t layer, const void* new_vals, int64_t seq_len,
                                 const int32_t* block_tables, int64_t n_layers, int64_t batch,
                                 int64_t max_blocks_per_seq, const int32_t* start_positions, void* stream) {
  int rb = 0;
  FMOE_TRY(kv_common(cache, dtype, n_blocks, block_size, n_head_kv, head_dim, &rb));
  FMOE_TRY(check_dims("n_layers", n_layers, 1, kMaxDim));
  FMOE_TRY(check_dims("layer", layer, 0, n_layers - 1));
  FMOE_TRY(check_dims("batch", batch, 0, 65535));
  FMOE_TRY(check_dims("seq_len", seq_len, 0, kMaxDim));
  FMOE_TRY(check_dims("max_blocks_per_seq", max_blocks_per_seq, 1, kMaxDim));
  if (batch == 0 || seq_len == 0) return ok();
  if (!new_vals || !block_tables || !start_positions) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (reinterpret_cast<uintptr_t>(new_vals) % 4) return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned new_vals");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_kv_scatter_prefill(cache, n_blocks, static_cast<int>(block_size), rb, new_vals,
                                     static_cast<int>(seq_len), block_tables + layer * batch * max_blocks_per_seq,
                                     static_cast<int>(max_blocks_per_seq), start_positions, static_cast<int>(batch),
                                     static_cast<hipStream_t>(stream)));
  return ok();
}

// ------------------------------------------------------------ dense linear weights
int fmoe_pack_linear_weight(const void* src, int src_dtype, int64_t n_in, int64_t n_out, int64_t row_offset,
                            int64_t n_out_total, int dst_dtype, void* dst, float* dst_scales, void* stream) {
  if (src_dtype != FMOE_F32 && src_dtype != FMOE_BF16) return fail(FMOE_ERR_DTYPE, "source dtype %d", src_dtype);
  if (!w_dtype_ok(dst_dtype)) return fail(FMOE_ERR_DTYPE, "packed dtype %d", dst_dtype);
  FMOE_TRY(check_dims("n_in", n_in, 0, kMaxDim));
  FMOE_TRY(check_dims("n_out_total", n_out_total, 0, kMaxDim));
  FMOE_TRY(check_dims("n_out", n_out, 0, n_out_total));
  FMOE_TRY(check_dims("row_offset", row_offset, 0, n_out_total - n_out));
  if (n_out == 0 || n_in == 0) return ok();
  if (!src || !dst) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (dst_dtype == FMOE_F8E4M3FN && !dst_scales) return fail(FMOE_ERR_INVALID_ARGUMENT, "fp8 needs dst_scales");
  FMOE_TRY(ensure_device());
  FMOE_HIP(launch_pack_linear(src, src_dtype, static_cast<int>(n_in), static_cast<int>(n_out),
                              static_cast<int>(row_offset), static_cast<int>(n_out_total), dst_dtype, dst, dst_scales,
                              static_cast<hipStream_t>(stream)));
  return ok();
}

// ------------------------------------------------------------ attention_block_decode
size_t fmoe_attention_block_decode_workspace_bytes(int64_t batch, int64_t ctx_len, int64_t n_head, int64_t n_head_kv,
                                                   int64_t n_embd, int64_t n_embd_kv, int act_dtype) {
  if (!act_dtype_ok(act_dtype) || batch < 0 || ctx_len < 0 || ctx_len > kMaxDim || n_head < 1 || n_head_kv < 1 ||
      n_embd < n_head || n_embd_kv < 0)
    return 0;
  const AttnShape a{batch, n_head, n_head_kv, n_embd, n_embd_kv, n_embd / n_head};
  return attn_layout(a, ctx_len, act_dtype).total;
}

int fmoe_attention_block_decode(const void* input, const int64_t* positions, const void* k_cached,
                                const void* v_cached, int64_t ctx_len, const void* packed_wqkv,
                                const float* wqkv_scales, const void* packed_wo, const float* wo_scales, int w_dtype,
                                const float* bq, const float* bk, const float* bv, const float* bo, int use_bias,
                                int64_t batch, int64_t n_head, int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv,
                                float rope_freq_base, float rope_freq_scale, int act_dtype, void* out, void* k_new,
                                void* v_new, void* workspace, size_t workspace_bytes, void* stream) {
  if (n_head < 1 || n_embd < 1) return fail(FMOE_ERR_SHAPE, "n_head and n_embd must be positive");
  const AttnShape a{batch, n_head, n_head_kv, n_embd, n_embd_kv, n_embd / n_head};
  FMOE_TRY(validate_attn_shape(a, act_dtype, w_dtype));
  FMOE_TRY(check_dims("ctx_len", ctx_len, 0, kMaxDim));
  const AttnWeights w{packed_wqkv, wqkv_scales, packed_wo, wo_scales, w_dtype, bq, bk, bv, bo, use_bias,
                      rope_freq_base, rope_freq_scale};
  FMOE_TRY(check_attn_weights(w));
  if (batch == 0) return ok();
  if (!input || !positions || !out || !k_new || !v_new || !workspace)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (ctx_len > 0 && (!k_cached || !v_cached)) return fail(FMOE_ERR_INVALID_ARGUMENT, "null cached K/V");
  if (ctx_len > 0 && (reinterpret_cast<uintptr_t>(k_cached) % 16 || reinterpret_cast<uintptr_t>(v_cached) % 16))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "cached K/V must be 16-byte aligned");
  if (batch * ctx_len > kMaxDim) return fail(FMOE_ERR_SHAPE, "batch * ctx_len exceeds 2^31-1");
  if (!aligned_for(input, act_dtype) || !aligned_for(out, act_dtype) || !aligned_for(k_new, act_dtype) ||
      !aligned_for(v_new, act_dtype))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  const AttnLayout L = attn_layout(a, ctx_len, act_dtype);
  FMOE_TRY(check_workspace(workspace, workspace_bytes, L.total));
  FMOE_TRY(ensure_device());
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The gathered [B, ctx, Hkv, D] tensors are a pool of B blocks of ctx rows,
  // sequence b owning block b in full.
  int* tables = at<int>(workspace, L.tables);
  int* lens = at<int>(workspace, L.lens);
  FMOE_HIP(launch_iota(tables, static_cast<int>(batch), nullptr, 0, 0, s));
  FMOE_HIP(launch_fill_int(lens, static_cast<int>(batch), static_cast<int>(ctx_len), s));
  FMOE_TRY(run_attention(a, w, input, positions, k_cached, v_cached, batch, static_cast<int>(ctx_len), tables, 1, lens,
                         static_cast<int>(ctx_len), act_dtype, out, k_new, v_new, workspace, L, s));
  return ok();
}

size_t fmoe_attention_decode_paged_workspace_bytes(int64_t batch, int64_t max_context_len, int64_t n_head,
                                                   int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv,
                                                   int act_dtype) {
  return fmoe_attention_block_decode_workspace_bytes(batch, max_context_len, n_head, n_head_kv, n_embd, n_embd_kv,
                                                     act_dtype);
}

static int attention_paged(const void* input, const void* residual, const void* norm_w, float rms_eps,
                           const int64_t* positions, void* k_cache, void* v_cache, int64_t n_blocks,
                           int64_t block_size, int64_t layer, const int32_t* block_tables,
                           const int32_t* context_lens, int64_t n_layers, int64_t max_blocks_per_seq,
                           int64_t max_context_len, const int32_t* block_indices, const int32_t* pos_in_blocks,
                           const void* packed_wqkv, const float* wqkv_scales, const void* packed_wo,
                           const float* wo_scales, int w_dtype, const float* bq, const float* bk, const float* bv,
                           const float* bo, int use_bias, int64_t batch, int64_t n_head, int64_t n_head_kv,
                           int64_t n_embd, int64_t n_embd_kv, float rope_freq_base, float rope_freq_scale,
                           int act_dtype, void* out, void* k_new, void* v_new, void* workspace,
                           size_t workspace_bytes, void* stream);

int fmoe_attention_decode_paged(const void* input, const int64_t* positions, void* k_cache, void* v_cache,
                                int64_t n_blocks, int64_t block_size, int64_t layer, const int32_t* block_tables,
                                const int32_t* context_lens, int64_t n_layers, int64_t max_blocks_per_seq,
                                int64_t max_context_len, const int32_t* block_indices, const int32_t* pos_in_blocks,
                                const void* packed_wqkv, const float* wqkv_scales, const void* packed_wo,
                                const float* wo_scales, int w_dtype, const float* bq, const float* bk,
                                const float* bv, const float* bo, int use_bias, int64_t batch, int64_t n_head,
                                int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv, float rope_freq_base,
                                float rope_freq_scale, int act_dtype, void* out, void* k_new, void* v_new,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return attention_paged(input, nullptr, nullptr, 0.f, positions, k_cache, v_cache, n_blocks, block_size, layer,
                         block_tables, context_lens, n_layers, max_blocks_per_seq, max_context_len, block_indices,
                         pos_in_blocks, packed_wqkv, wqkv_scales, packed_wo, wo_scales, w_dtype, bq, bk, bv, bo,
                         use_bias, batch, n_head, n_head_kv, n_embd, n_embd_kv, rope_freq_base, rope_freq_scale,
                         act_dtype, out, k_new, v_new, workspace, workspace_bytes, stream);
}

size_t fmoe_attention_sublayer_decode_paged_workspace_bytes(int64_t batch, int64_t max_context_len, int64_t n_head,
                                                            int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv,
                                                            int act_dtype) {
  const size_t base = fmoe_attention_block_decode_workspace_bytes(batch, max_context_len, n_head, n_head_kv, n_embd,
                                                                  n_embd_kv, act_dtype);
  if (base == 0) return 0;
  return base + align_up(static_cast<size_t>(batch) * n_embd * dtype_bytes(act_dtype));
}

int fmoe_attention_sublayer_decode_paged(const void* residual, const void* attn_norm_w, float rms_eps,
                                         const int64_t* positions, void* k_cache, void* v_cache, int64_t n_blocks,
                                         int64_t block_size, int64_t layer, const int32_t* block_tables,
                                         const int32_t* context_lens, int64_t n_layers, int64_t max_blocks_per_seq,
                                         int64_t max_context_len, const int32_t* block_indices,
                                         const int32_t* pos_in_blocks, const void* packed_wqkv,
                                         const float* wqkv_scales, const void* packed_wo, const float* wo_scales,
                                         int w_dtype, const float* bq, const float* bk, const float* bv,
                                         const float* bo, int use_bias, int64_t batch, int64_t n_head,
                                         int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv, float rope_freq_base,
                                         float rope_freq_scale, int act_dtype, void* out, void* k_new, void* v_new,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (batch > 0 && (!residual || !attn_norm_w)) return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (batch > 0 && !aligned_for(attn_norm_w, act_dtype)) return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  return attention_paged(residual, residual, attn_norm_w, rms_eps, positions, k_cache, v_cache, n_blocks, block_size,
                         layer, block_tables, context_lens, n_layers, max_blocks_per_seq, max_context_len,
                         block_indices, pos_in_blocks, packed_wqkv, wqkv_scales, packed_wo, wo_scales, w_dtype, bq,
                         bk, bv, bo, use_bias, batch, n_head, n_head_kv, n_embd, n_embd_kv, rope_freq_base,
                         rope_freq_scale, act_dtype, out, k_new, v_new, workspace, workspace_bytes, stream);
}

}  // extern "C"

// Shared by the paged attention and the attention sub-layer: norm_w non-null
// normalises `input` into the workspace first (attn_norm,
// transformer_layer_moe_decode.mlir:174-177) and `residual` is added to the
// output (:208-221).
static int attention_paged(const void* input, const void* residual, const void* norm_w, float rms_eps,
                           const int64_t* positions, void* k_cache, void* v_cache, int64_t n_blocks,
                           int64_t block_size, int64_t layer, const int32_t* block_tables,
                           const int32_t* context_lens, int64_t n_layers, int64_t max_blocks_per_seq,
                           int64_t max_context_len, const int32_t* block_indices, const int32_t* pos_in_blocks,
                           const void* packed_wqkv, const float* wqkv_scales, const void* packed_wo,
                           const float* wo_scales, int w_dtype, const float* bq, const float* bk, const float* bv,
                           const float* bo, int use_bias, int64_t batch, int64_t n_head, int64_t n_head_kv,
                           int64_t n_embd, int64_t n_embd_kv, float rope_freq_base, float rope_freq_scale,
                           int act_dtype, void* out, void* k_new, void* v_new, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (n_head < 1 || n_embd < 1) return fail(FMOE_ERR_SHAPE, "n_head and n_embd must be positive");
  const AttnShape a{batch, n_head, n_head_kv, n_embd, n_embd_kv, n_embd / n_head};
  FMOE_TRY(validate_attn_shape(a, act_dtype, w_dtype));
  FMOE_TRY(check_pool(n_blocks, block_size));
  FMOE_TRY(check_dims("n_layers", n_layers, 1, kMaxDim));
  FMOE_TRY(check_dims("layer", layer, 0, n_layers - 1));
  FMOE_TRY(check_dims("max_blocks_per_seq", max_blocks_per_seq, 1, kMaxDim));
  FMOE_TRY(check_dims("max_context_len", max_context_len, 0, kMaxDim));
  const AttnWeights w{packed_wqkv, wqkv_scales, packed_wo, wo_scales, w_dtype, bq, bk, bv, bo, use_bias,
                      rope_freq_base, rope_freq_scale};
  FMOE_TRY(check_attn_weights(w));
  if (batch == 0) return ok();
  if (!input || !positions || !k_cache || !v_cache || !block_tables || !context_lens || !block_indices ||
      !pos_in_blocks || !out || !workspace)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "null pointer");
  if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16)
    return fail(FMOE_ERR_INVALID_ARGUMENT, "K/V pools must be 16-byte aligned");
  if (!aligned_for(input, act_dtype) || !aligned_for(out, act_dtype) || (k_new && !aligned_for(k_new, act_dtype)) ||
      (v_new && !aligned_for(v_new, act_dtype)))
    return fail(FMOE_ERR_INVALID_ARGUMENT, "misaligned pointer");
  const AttnLayout L = attn_layout(a, max_context_len, act_dtype);
  const size_t xn_off = L.total;
  const size_t need = norm_w ? xn_off + align_up(static_cast<size_t>(batch) * n_embd * dtype_bytes(act_dtype))
                             : L.total;
  FMOE_TRY(check_workspace(workspace, workspace_bytes, need));
  FMOE_TRY(ensure_device());
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* kn = k_new ? k_new : at<char>(workspace, L.k_new);
  void* vn = v_new ? v_new : at<char>(workspace, L.v_new);
  const void* x = input;
  if (norm_w) {
    void* xn = at<char>(workspace, xn_off);
    ScopedTimer t(FMOE_TIMER_NORM, s);
    FMOE_HIP(launch_rms_norm(input, norm_w, rms_eps, xn, batch, static_cast<int>(n_embd), act_dtype, s));
    x = xn;
  }
  // scatter_decode once the attention has read the pools
  // (transformer_layer_moe_decode.mlir:202-206), in the combine launch.
  KvScatterDecode sc;
  sc.k_cache = k_cache;
  sc.v_cache = v_cache;
  sc.n_blocks = n_blocks;
  sc.block_size = static_cast<int>(block_size);
  sc.row_bytes = static_cast<int>(n_embd_kv * dtype_bytes(act_dtype));
  sc.block_idx = block_indices;
  sc.pos_idx = pos_in_blocks;
  FMOE_TRY(run_attention(a, w, x, positions, k_cache, v_cache, n_blocks, static_cast<int>(block_size),
                         block_tables + layer * batch * max_blocks_per_seq, static_cast<int>(max_blocks_per_seq),
                         context_lens + layer * batch, static_cast<int>(max_context_len), act_dtype, out, kn, vn,
                         workspace, L, s, residual, &sc));
  return ok();
}
