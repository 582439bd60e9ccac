// C ABI of libveymoe: argument validation, workspace layout, launch order and
// per-kernel event timing.  Shape contracts follow MetalMoEExecutor
// (models/flashnext/metal_runtime.py:430-461 and :837-895); status codes and
// the thread-local last error follow the reference's native executor
// (models/flashnext/tests/bench/metal_runtime_native.mm:196-209).

#include <hip/hip_runtime.h>

#include <atomic>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/veymoe.h"
#include "vm_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(VM_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr uint32_t kMaxTopK = 10;       // MAX_TOP_K, metal_runtime.py:28
constexpr uint32_t kMaxExperts = 512;   // MAX_EXPERTS, metal_runtime.py:27
constexpr uint32_t kMaxWidth = 16384;   // MAX_WIDTH, metal_runtime.py:29
constexpr uint64_t kAlign = 256;

uint64_t align_up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
uint32_t act_bytes(uint32_t dtype) { return dtype == VM_BF16 ? 2u : 4u; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

vm::ProjPtrs to_ptrs(const VmQ4Proj& q) { return vm::ProjPtrs{q.weight, q.scales, q.biases}; }

vm::PoolDev to_pool(const VmPoolView& v) {
  vm::PoolDev d{};
  d.base = v.base;
  d.header = v.header_size;
  d.stride = v.record_stride;
  for (int i = 0; i < VM_PARTS; ++i) d.off[i] = v.part_offset[i];
  d.records = v.base != nullptr ? v.records : 0;
  return d;
}

bool proj_ok(const VmQ4Proj& q) {
  if (q.weight == nullptr) return q.scales == nullptr && q.biases == nullptr;
  return q.scales != nullptr && q.biases != nullptr && aligned16(q.weight);
}

int check_pool(const VmPoolView& v, uint32_t hidden, uint32_t inter) {
  if (v.base == nullptr) return VM_OK;
  // every part must fit inside the record and keep 16-byte alignment of the words
  const uint64_t sizes[VM_PARTS] = {
      uint64_t(inter) * hidden / 2, uint64_t(inter) * (hidden / 32) * 2, uint64_t(inter) * (hidden / 32) * 2,
      uint64_t(inter) * hidden / 2, uint64_t(inter) * (hidden / 32) * 2, uint64_t(inter) * (hidden / 32) * 2,
      uint64_t(hidden) * inter / 2, uint64_t(hidden) * (inter / 32) * 2, uint64_t(hidden) * (inter / 32) * 2};
  for (int i = 0; i < VM_PARTS; ++i) {
    if (v.part_offset[i] + sizes[i] > v.record_stride)
      return fail(VM_EINVAL, "pool part %d (offset %llu, %llu bytes) exceeds the record stride %llu", i,
                  (unsigned long long)v.part_offset[i], (unsigned long long)sizes[i],
                  (unsigned long long)v.record_stride);
  }
  const uint64_t wparts[3] = {v.part_offset[0], v.part_offset[3], v.part_offset[6]};
  for (uint64_t off : wparts)
    if ((v.header_size + off) % 16 || v.record_stride % 16)
      return fail(VM_EINVAL, "pool weight parts must be 16-byte aligned");
  if (!aligned16(v.base)) return fail(VM_EINVAL, "pool base must be 16-byte aligned");
  return VM_OK;
}

// ------------------------------------------------------------ timing ----

struct Timing {
  std::mutex mu;
  bool enabled = false;
  struct Pending {
    hipEvent_t start, end;
  };
  std::map<std::string, std::vector<Pending>> pending;
  std::map<std::string, std::pair<double, uint64_t>> totals;
  std::vector<hipEvent_t> free_events;

  hipEvent_t get() {
    if (!free_events.empty()) {
      hipEvent_t e = free_events.back();
      free_events.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};

Timing& timing() {
  static Timing t;
  return t;
}

int drain_timing(Timing& t) {
  for (auto& kv : t.pending) {
    auto& tot = t.totals[kv.first];
    for (auto& pe : kv.second) {
      hipError_t e = hipEventSynchronize(pe.end);
      if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
      float ms = 0.0f;
      e = hipEventElapsedTime(&ms, pe.start, pe.end);
      if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
      tot.first += ms;
      tot.second += 1;
      t.free_events.push_back(pe.start);
      t.free_events.push_back(pe.end);
    }
    kv.second.clear();
  }
  return VM_OK;
}

}  // namespace

namespace vm {

bool timing_events(const char* family, hipEvent_t* start, hipEvent_t* stop) {
  Timing& t = timing();
  if (!t.enabled) return false;
  std::lock_guard<std::mutex> lock(t.mu);
  hipEvent_t s = t.get();
  hipEvent_t e = t.get();
  if (s == nullptr || e == nullptr) return false;
  t.pending[family].push_back({s, e});
  *start = s;
  *stop = e;
  return true;
}

}  // namespace vm

// The workspace of vm_moe_layer_static: one array per device in the library's
// own device memory, held until the process ends.  On the host, `scratch`
// names a stand-in, not a device address: host code uses only the address
// that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[VM_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// This device's scratch address, looked up once per device with the device
// current.
int scratch_address(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(VM_EUNSUPPORTED, "device %d is beyond the scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t s = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (s != hipSuccess) return hip_fail(s, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(VM_EHIP, "hipGetSymbolAddress(scratch) returned no address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return VM_OK;
}

// A second stream of the calling thread on the current device, for the part
// of a grouped layer call that does not depend on the routing (the shared
// expert): forked from the caller's stream with one event and joined back
// with another before the combine, so it runs beside the router GEMM, the
// selection and the sort, which leave most of the GPU idle.  Created on the
// thread's first such call on the device (never while the caller's stream is
// being captured, and never for vm_moe_layer_static, whose callers cannot
// allocate) and held until the process ends.  Without it the call takes the
// one-stream path, with the same results.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
thread_local bool t_static_call = false;

SideStream* side_stream(hipStream_t caller) {
  thread_local SideStream per_device[kMaxDevices];
  if (t_static_call) return nullptr;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  SideStream& s = per_device[dev];
  if (s.stream == nullptr) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(caller, &status) != hipSuccess || status != hipStreamCaptureStatusNone) return nullptr;
    SideStream n;
    if (hipStreamCreateWithFlags(&n.stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&n.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&n.join, hipEventDisableTiming) != hipSuccess) {
      if (n.join != nullptr) (void)hipEventDestroy(n.join);
      if (n.fork != nullptr) (void)hipEventDestroy(n.fork);
      if (n.stream != nullptr) (void)hipStreamDestroy(n.stream);
      (void)hipGetLastError();
      return nullptr;
    }
    s = n;
  }
  return &s;
}

}  // namespace

extern "C" {

int vm_abi_version(void) { return VM_ABI_VERSION; }

int vm_available(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    fail(VM_EHIP, "no HIP device is visible");
    return 0;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    fail(VM_EUNSUPPORTED, "device %d is %s; this library is built for gfx950", dev, prop.gcnArchName);
    return 0;
  }
  return 1;
}

int vm_last_error(char* buf, size_t len) {
  if (buf == nullptr || len == 0) return VM_EINVAL;
  std::strncpy(buf, g_last_error.c_str(), len - 1);
  buf[len - 1] = '\0';
  return VM_OK;
}

// ------------------------------------------------------------ execute ---

uint64_t vm_moe_execute_workspace(uint32_t tokens, uint32_t slots, uint32_t inter_size, uint32_t act_dtype) {
  return align_up(uint64_t(tokens) * slots * inter_size * act_bytes(act_dtype)) + kAlign;
}

int vm_moe_execute(const VmMoeArgs* a, void* stream_ptr) {
  if (a == nullptr) return fail(VM_EINVAL, "null arguments");
  const hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const uint32_t T = a->tokens, K = a->slots, H = a->hidden_size, I = a->inter_size;
  if (a->act_dtype > VM_F32 || a->score_dtype > VM_F32) return fail(VM_EINVAL, "unknown dtype");
  if (a->group_size != 32) return fail(VM_EUNSUPPORTED, "group_size must be 32");
  if (T == 0) return fail(VM_EINVAL, "tokens must be positive");
  if (K == 0 || K > kMaxTopK) return fail(VM_EINVAL, "slots must be in 1..%u", kMaxTopK);
  if (a->expert_count == 0 || a->expert_count > 0x7fffffffu) return fail(VM_EINVAL, "expert_count must be positive");
  if (H == 0 || I == 0 || H % 32 || I % 32)
    return fail(VM_EINVAL, "Q4/G32 projection inputs must be group aligned");
  if (I > kMaxWidth) return fail(VM_EINVAL, "gate and up projection widths must match the bound");
  if (a->x == nullptr || a->routes == nullptr) return fail(VM_EINVAL, "x and routes are required");
  if (a->output == nullptr && a->activation_out == nullptr)
    return fail(VM_EINVAL, "an output or an activation output is required");
  if (a->output == nullptr && a->activation_in != nullptr)
    return fail(VM_EINVAL, "precomputed activations need an output");
  if (!aligned16(a->x) || (a->activation_in && !aligned16(a->activation_in)))
    return fail(VM_EINVAL, "activations must be 16-byte aligned");
  if ((a->shared == nullptr) != (a->shared_gate == nullptr))
    return fail(VM_EINVAL, "shared and shared_gate must be provided together");
  if (a->shared_y != nullptr && a->shared != nullptr)
    return fail(VM_EINVAL, "provide shared_y or shared parts, not both");
  if (a->scores == nullptr && (a->shared_y != nullptr || a->shared != nullptr))
    return fail(VM_EINVAL, "a shared term needs scores");
  if (!proj_ok(a->gate) || !proj_ok(a->up) || !proj_ok(a->down))
    return fail(VM_EINVAL, "projection weight, scales and biases must be given together (weights 16-byte aligned)");
  if (a->pool.base == nullptr && a->gate.weight == nullptr && a->stream.base == nullptr)
    return fail(VM_EINVAL, "neither dense projections nor a pool view was given");
  if (a->slot_table != nullptr && a->pool.base == nullptr)
    return fail(VM_EINVAL, "a slot table needs a pool view");
  if (a->stream.base != nullptr && a->pool.base == nullptr)
    return fail(VM_EINVAL, "stream pack requires a resident slab pack");
  int rc = check_pool(a->pool, H, I);
  if (rc != VM_OK) return rc;
  rc = check_pool(a->stream, H, I);
  if (rc != VM_OK) return rc;
  if (!vm::gateup_supported(H)) return fail(VM_EUNSUPPORTED, "hidden_size %u is above the decode kernel bound", H);
  if (!vm::down_supported(I, K, a->act_dtype))
    return fail(VM_EUNSUPPORTED, "inter_size %u with %u slots is above the decode kernel bound", I, K);

  const uint64_t need = vm_moe_execute_workspace(T, K, I, a->act_dtype);
  void* act = const_cast<void*>(a->activation_in);
  if (act == nullptr) {
    act = a->activation_out;
    if (act == nullptr) {
      if (a->workspace == nullptr || a->workspace_bytes < need)
        return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)need);
      act = a->workspace;
    }
    vm::GateUpLaunch g{};
    g.x = a->x;
    g.routes = a->routes;
    g.slot_table = a->slot_table;
    g.gate = to_ptrs(a->gate);
    g.up = to_ptrs(a->up);
    g.pool = to_pool(a->pool);
    g.stream = to_pool(a->stream);
    g.act = act;
    g.gate_out = a->gate_out;
    g.up_out = a->up_out;
    g.status = a->status;
    g.tokens = T;
    g.slots = K;
    g.hidden = H;
    g.inter = I;
    g.experts = a->expert_count;
    g.has_shared = 0;
    g.act_dtype = static_cast<int>(a->act_dtype);
    hipError_t e = vm::launch_gateup(g, stream);
    if (e != hipSuccess) return hip_fail(e, "gate/up launch");
  }
  if (a->output == nullptr) return VM_OK;
  vm::DownLaunch d{};
  d.act = act;
  d.routes = a->routes;
  d.slot_table = a->slot_table;
  d.down = to_ptrs(a->down);
  d.pool = to_pool(a->pool);
  d.stream = to_pool(a->stream);
  d.scores = a->scores;
  d.score_dtype = static_cast<int>(a->score_dtype);
  d.shared_y = a->shared_y;
  d.shared = a->shared;
  d.shared_gate = a->shared_gate;
  d.out = a->output;
  d.status = a->status;
  d.tokens = T;
  d.slots = K;
  d.hidden = H;
  d.inter = I;
  d.experts = a->expert_count;
  d.has_shared = 0;
  d.act_dtype = static_cast<int>(a->act_dtype);
  hipError_t e = vm::launch_down(d, stream);
  if (e != hipSuccess) return hip_fail(e, "down launch");
  return VM_OK;
}

// ------------------------------------------------------------- router ---

uint64_t vm_router_workspace(uint32_t tokens, uint32_t expert_count) {
  return kAlign + align_up(uint64_t(tokens) * expert_count * 4);
}

static int validate_router(uint32_t T, uint32_t H, uint32_t E, uint32_t K, uint32_t dtype) {
  if (dtype > VM_F32) return fail(VM_EINVAL, "unknown dtype");
  if (T == 0) return fail(VM_EINVAL, "tokens must be positive");
  if (E == 0 || E > kMaxExperts) return fail(VM_EINVAL, "expert_count must be in 1..%u", kMaxExperts);
  if (K == 0 || K > kMaxTopK) return fail(VM_EINVAL, "top_k must be in 1..%u", kMaxTopK);
  if (K > E) return fail(VM_EINVAL, "top_k cannot exceed expert_count");
  if (H == 0 || H % 32) return fail(VM_EINVAL, "hidden_size must be a positive multiple of 32");
  if (H > 8192) return fail(VM_EUNSUPPORTED, "hidden_size %u is above the router kernel bound (8192)", H);
  return VM_OK;
}

int vm_router_topk(const VmRouterArgs* a, void* stream_ptr) {
  if (a == nullptr) return fail(VM_EINVAL, "null arguments");
  int rc = validate_router(a->tokens, a->hidden_size, a->expert_count, a->top_k, a->act_dtype);
  if (rc != VM_OK) return rc;
  if (a->x == nullptr || a->weight == nullptr || a->inds == nullptr || a->scores == nullptr)
    return fail(VM_EINVAL, "x, weight, inds and scores are required");
  if (!aligned16(a->x) || !aligned16(a->weight)) return fail(VM_EINVAL, "x and weight must be 16-byte aligned");
  const uint64_t need = vm_router_workspace(a->tokens, a->expert_count);
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)need);
  const hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  float* logits = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + kAlign);
  vm::FrontLaunch f{};
  f.x = a->x;
  f.weight = a->weight;
  f.bias = a->logit_bias;
  f.logits = logits;
  f.tokens = a->tokens;
  f.hidden = a->hidden_size;
  f.experts = a->expert_count;
  f.act_dtype = static_cast<int>(a->act_dtype);
  hipError_t e = vm::launch_front(f, stream);
  if (e != hipSuccess) return hip_fail(e, "router launch");
  vm::SelectLaunch s{};
  s.logits = logits;
  s.inds = a->inds;
  s.scores = a->scores;
  s.gates = a->gates;
  s.tokens = a->tokens;
  s.experts = a->expert_count;
  s.top_k = a->top_k;
  s.act_dtype = static_cast<int>(a->act_dtype);
  s.blend = a->renorm_blend;
  e = vm::launch_select(s, stream);
  if (e != hipSuccess) return hip_fail(e, "select launch");
  return VM_OK;
}

// -------------------------------------------------------------- layer ---
// workspace: [reserved] [logits T*E f32] [act T*S*I] [sig T] [inds T*K] [scores T*K] [words T*K]
//            [fill list of the device LRU: count, source rows, slots]

struct LayerWs {
  uint64_t logits, act, sig, inds, scores, words, fill, tags, total;
};

static LayerWs layer_ws(uint32_t T, uint32_t K, uint32_t I, uint32_t Is, uint32_t E, uint32_t dtype) {
  LayerWs w{};
  const uint32_t S = K + (Is ? 1 : 0);
  w.logits = kAlign;
  w.act = w.logits + align_up(uint64_t(T) * E * 4);
  w.sig = w.act + align_up(uint64_t(T) * S * I * act_bytes(dtype));
  w.inds = w.sig + align_up(uint64_t(T) * act_bytes(dtype));
  w.scores = w.inds + align_up(uint64_t(T) * K * 4);
  w.words = w.scores + align_up(uint64_t(T) * K * act_bytes(dtype));
  w.fill = w.words + align_up(uint64_t(T) * K * 4);
  w.tags = w.fill + align_up(4 + 8 * uint64_t(vm::kLruMaxRouted));
  // hand-off words of the two-launch one-token pipeline (built on request):
  // one-token bf16 calls are the only ones it takes
  w.total = w.tags + (VM_FUSED_PIPELINES && T == 1 && dtype == VM_BF16 ? align_up(vm::tag_words(K * I) * 4) : 0);
  return w;
}

// -------------------------------------------------------- fused decode ---
// The decode pipeline of one-token calls, process-wide:
//   0  k_front, k_gateup (routed + shared pairs), k_down (the default: the
//      fastest measured, 14.6 us per layer against 16.1 and 21.4 at hidden
//      2048 / inter 512 / 512 experts top-10 + shared);
//   1  the one-token front (router + shared expert gate/up), the gate/up grid
//      of a block per CU, k_down;
//   2  the one-token front and the experts grid with the tagged hand-off.
static std::atomic<int> g_fused_decode{0};

// Compute units of the current device: the experts grid is one block per CU
// so that all of it is resident at once.
static uint32_t device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 0;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return static_cast<uint32_t>(v);
}

static vm::Inject to_inject(const VmLayerArgs* a) {
  vm::Inject j{};
  if (a->inject_out != nullptr) {
    j.hidden = a->inject_hidden;
    j.weights = a->inject_weights;
    j.out = a->inject_out;
    j.hc = a->hc_count;
  }
  return j;
}

// The fused launch arguments of a one-token bf16 call, or false when the
// three-launch path serves it.
static bool fused_args(const VmLayerArgs* a, const LayerWs& w, char* ws, vm::FusedLaunch& f, uint32_t& blocks,
                       bool& two_launch) {
  const int mode = g_fused_decode.load(std::memory_order_relaxed);
  if (mode == 0) return false;
  two_launch = mode == 2;
  if (a->tokens != 1 || a->act_dtype != VM_BF16) return false;
  blocks = device_cus();
  const uint32_t K = a->top_k, I = a->inter_size, H = a->hidden_size;
  const bool shared = a->shared_inter != 0;
  f = vm::FusedLaunch{};
  if (!vm::fused_plan(H, I, K, shared ? 1u : 0u, a->expert_count, blocks, f)) return false;
  f.x = static_cast<const uint16_t*>(a->x);
  f.router = a->router_weight;
  f.router_bias = a->router_bias;
  f.logits = reinterpret_cast<float*>(ws + w.logits);
  if (shared) {
    f.sh_gate = to_ptrs(a->shared_gate_proj);
    f.sh_up = to_ptrs(a->shared_up_proj);
    f.sh_down = to_ptrs(a->shared_down_proj);
    f.sh_seg = to_ptrs(a->shared_expert_gate);
  }
  // activations [K + 1, I]: routed slots, then the shared expert's
  f.act = reinterpret_cast<uint16_t*>(ws + w.act);
  f.sh_act = f.act + uint64_t(K) * I;
  f.sh_sig = reinterpret_cast<uint16_t*>(ws + w.sig);
  f.slot_table = a->slot_table;
  f.pool = to_pool(a->pool);
  f.gate = to_ptrs(a->gate);
  f.up = to_ptrs(a->up);
  f.down = to_ptrs(a->down);
  f.act_tag = two_launch ? reinterpret_cast<uint32_t*>(ws + w.tags) : nullptr;
  f.words_out = reinterpret_cast<uint32_t*>(ws + w.words);
  f.out = static_cast<uint16_t*>(a->output);
  f.inds_out = a->inds_out != nullptr ? a->inds_out : reinterpret_cast<int32_t*>(ws + w.inds);
  f.scores_out = static_cast<uint16_t*>(a->scores_out != nullptr ? a->scores_out : static_cast<void*>(ws + w.scores));
  f.status = a->status;
  f.inject = to_inject(a);
  f.hidden = H;
  f.inter = I;
  f.experts = a->expert_count;
  f.slots = K;
  f.has_shared = shared ? 1u : 0u;
  f.generic = a->combine == VM_COMBINE_GENERIC ? 1u : 0u;
  f.blend = a->renorm_blend;
  return true;
}

// Workspace of the grouped path (more than VM_LAYER_MAX_TOKENS rows).
struct GroupedWs {
  uint64_t logits, sig, inds, scores, row_off, tiles, tile_count, tiles_dn, tile_count_dn, sort_counts,
      sort_cursors, row_token, pair_row, act, rows, total;
  uint32_t rows_total, groups, max_tiles, max_tiles_dn, tile_rows, tile_rows_dn;
  bool small;  // 16-row tile kernels (k_rows)
};

// Calls of up to this many tokens run the 16-row tile kernels, whose blocks
// stage their tile's A rows once and stream the weights without barriers:
// with few rows per expert the chunked GEMM's 64-row tiles ran mostly empty.
constexpr uint32_t kRowsMaxTokens = 64;

#ifndef VM_ROWS_PATH
#define VM_ROWS_PATH 1
#endif
// Router logits of calls above 64 rows: the LDS-ring bf16 GEMM (1) or the
// chunked GEMM shared with the Q4 projections (0).
#ifndef VM_ROUTER_RING
#define VM_ROUTER_RING 1
#endif
static bool small_grouped(uint32_t T, uint32_t H, uint32_t I) {
  return VM_ROWS_PATH && T <= kRowsMaxTokens && vm::rows_supported(H) && vm::rows_supported(I);
}

// Rows per gate/up tile of a chunked-GEMM call: tall tiles when the routed
// experts average more rows than one tile of the usual height holds and the
// hidden size is a whole number of K chunks (the tall instance has no tail
// chunk).  Measured at 512 experts top-10: 3584 rows 592-594 -> 546 us per
// call, 4096 rows 642-650 -> 581-589 us, no change at 2048 or 8192 rows.
static uint32_t gateup_tile_rows(uint32_t T, uint32_t K, uint32_t H, uint32_t E) {
  const bool tall = uint64_t(T) * K > uint64_t(E) * vm::kGroupedRows && H % (8 * 32) == 0;
  return tall ? vm::kGroupedRowsTall : vm::kGroupedRows;
}

// Rows per down tile: the same rule over the intermediate size and the down
// GEMM's usual height (3072 rows 514-519 -> 502-508 us per call).
static uint32_t down_tile_rows(uint32_t T, uint32_t K, uint32_t I, uint32_t E) {
  const bool tall = uint64_t(T) * K > uint64_t(E) * vm::kGroupedRowsDown && I % (8 * 32) == 0;
  return tall ? vm::kGroupedRowsTall : vm::kGroupedRowsDown;
}

static GroupedWs grouped_ws(uint32_t T, uint32_t K, uint32_t H, uint32_t I, uint32_t E, bool shared) {
  GroupedWs w{};
  w.rows_total = T * K + (shared ? T : 0);
  w.groups = E + (shared ? 1 : 0);
  w.small = small_grouped(T, H, I);
  w.tile_rows = w.small ? vm::kRowsTile : gateup_tile_rows(T, K, H, E);
  w.tile_rows_dn = w.small ? vm::kRowsTile : down_tile_rows(T, K, I, E);
  w.max_tiles = vm::grouped_max_tiles(w.rows_total, w.groups, w.tile_rows);
  w.max_tiles_dn = vm::grouped_max_tiles(w.rows_total, w.groups, w.tile_rows_dn);
  uint64_t o = kAlign;
  auto take = [&](uint64_t bytes) {
    const uint64_t at = o;
    o += align_up(bytes);
    return at;
  };
  w.logits = take(uint64_t(T) * E * 4);
  w.sig = take(uint64_t(T) * 2);
  w.inds = take(uint64_t(T) * K * 4);
  w.scores = take(uint64_t(T) * K * 2);
  w.row_off = take(uint64_t(w.groups + 1) * 4);
  w.tiles = take(uint64_t(w.max_tiles) * 8);
  w.tile_count = take(4);
  w.tiles_dn = take(uint64_t(w.max_tiles_dn) * 8);
  w.tile_count_dn = take(4);
  // the counts and the cursors of the multi-block sort, one region (the
  // router GEMM zeroes both in one pass when the select counts the rows)
  w.sort_counts = take(2048 * 4);
  w.sort_cursors = w.sort_counts + 1024 * 4;
  w.row_token = take(uint64_t(w.rows_total) * 4);
  w.pair_row = take(uint64_t(T) * K * 4);
  w.act = take(uint64_t(w.rows_total) * I * 2);
  w.rows = take(uint64_t(w.rows_total) * H * 2);
  w.total = o;
  return w;
}

static bool use_grouped(uint32_t T, uint32_t dtype) { return T > VM_LAYER_MAX_TOKENS && dtype == VM_BF16; }

// Up to this many rows the grouped layer keeps the decode router kernel (one
// router row per wave over every token); above, the router is an MFMA GEMM.
constexpr uint32_t kFrontMaxTokens = 64;

// Calls above this many rows run the shared expert on a side stream beside the
// router GEMM, the selection and the sort.  Its fork and join cost the caller's
// stream about 6 us each, which smaller calls do not win back: with the shared
// expert as one more group of the sorted GEMMs, 96 rows took 86 us instead of
// 93 and 256 rows 117 instead of 120, while 512 rows took 288 instead of 283
// and 2048 rows 386 instead of 382.
constexpr uint32_t kSideMinTokens = 256;

uint64_t vm_moe_layer_workspace(uint32_t tokens, uint32_t top_k, uint32_t hidden_size, uint32_t inter_size,
                                uint32_t shared_inter, uint32_t expert_count, uint32_t act_dtype) {
  if (use_grouped(tokens, act_dtype))
    return grouped_ws(tokens, top_k, hidden_size, inter_size, expert_count, shared_inter != 0).total;
  if (tokens <= VM_LAYER_MAX_TOKENS) return layer_ws(tokens, top_k, inter_size, shared_inter, expert_count, act_dtype).total;
  // fp32 above the decode bound: one decode workspace per chunk of
  // VM_LAYER_MAX_TOKENS rows, so that a router-only call leaves every chunk's
  // routes and shared gate for the experts-only call
  const uint64_t per = align_up(layer_ws(VM_LAYER_MAX_TOKENS, top_k, inter_size, shared_inter, expert_count,
                                         act_dtype).total);
  return per * ((tokens + VM_LAYER_MAX_TOKENS - 1) / VM_LAYER_MAX_TOKENS);
}

static int layer_decode(const VmLayerArgs* a, hipStream_t stream);
static int layer_grouped(const VmLayerArgs* a, hipStream_t stream);

static int validate_layer(const VmLayerArgs* a) {
  if (a == nullptr) return fail(VM_EINVAL, "null arguments");
  const uint32_t H = a->hidden_size, I = a->inter_size;
  int rc = validate_router(a->tokens, H, a->expert_count, a->top_k, a->act_dtype);
  if (rc != VM_OK) return rc;
  if (a->group_size != 32) return fail(VM_EUNSUPPORTED, "group_size must be 32");
  if (I == 0 || I % 32) return fail(VM_EINVAL, "Q4/G32 projection inputs must be group aligned");
  if (a->shared_inter != 0 && a->shared_inter != I)
    return fail(VM_EUNSUPPORTED, "shared_inter must be 0 or equal to inter_size");
  if (a->x == nullptr || a->output == nullptr || a->router_weight == nullptr)
    return fail(VM_EINVAL, "x, output and router_weight are required");
  if (!aligned16(a->x) || !aligned16(a->router_weight)) return fail(VM_EINVAL, "x and router weight must be 16-byte aligned");
  if (a->slot_table != nullptr && a->pool.base == nullptr) return fail(VM_EINVAL, "a slot table needs a pool view");
  if (a->slot_table == nullptr && a->gate.weight == nullptr)
    return fail(VM_EINVAL, "routed experts need a slot table with a pool view, or dense projections");
  if (!proj_ok(a->gate) || !proj_ok(a->up) || !proj_ok(a->down)) return fail(VM_EINVAL, "malformed routed projection");
  const bool shared = a->shared_inter != 0;
  if (shared) {
    if (a->shared_gate_proj.weight == nullptr || a->shared_up_proj.weight == nullptr ||
        a->shared_down_proj.weight == nullptr || a->shared_expert_gate.weight == nullptr)
      return fail(VM_EINVAL, "shared expert projections and its gate are required when shared_inter > 0");
    if (!proj_ok(a->shared_gate_proj) || !proj_ok(a->shared_up_proj) || !proj_ok(a->shared_down_proj) ||
        !proj_ok(a->shared_expert_gate))
      return fail(VM_EINVAL, "malformed shared projection");
  }
  rc = check_pool(a->pool, H, I);
  if (rc != VM_OK) return rc;
  const uint32_t phases = a->phases == 0 ? (VM_PHASE_ROUTER | VM_PHASE_EXPERTS) : a->phases;
  if (phases & ~(VM_PHASE_ROUTER | VM_PHASE_EXPERTS)) return fail(VM_EINVAL, "unknown phase bits");
  if (a->combine != VM_COMBINE_FUSED && a->combine != VM_COMBINE_GENERIC)
    return fail(VM_EINVAL, "combine must be VM_COMBINE_FUSED or VM_COMBINE_GENERIC");
  if (a->inject_out != nullptr) {
    if (a->inject_hidden == nullptr || a->inject_weights == nullptr)
      return fail(VM_EINVAL, "an injection needs inject_hidden and inject_weights");
    if (a->hc_count == 0 || a->hc_count > VM_MAX_STREAMS)
      return fail(VM_EINVAL, "hc_count must be 1..%d", VM_MAX_STREAMS);
    if (!aligned16(a->inject_hidden) || !aligned16(a->inject_out))
      return fail(VM_EINVAL, "inject_hidden and inject_out must be 16-byte aligned");
  }
  return VM_OK;
}

int vm_moe_layer(const VmLayerArgs* a, void* stream_ptr) {
  int rc = validate_layer(a);
  if (rc != VM_OK) return rc;
  const hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const uint32_t T = a->tokens, K = a->top_k, H = a->hidden_size;
  if (use_grouped(T, a->act_dtype)) return layer_grouped(a, stream);
  if (T <= VM_LAYER_MAX_TOKENS) return layer_decode(a, stream);
  // fp32 activations above the decode bound: decode kernels in chunks of
  // VM_LAYER_MAX_TOKENS tokens (with no rounding the fused and the generic
  // combine agree), each chunk in a workspace slice of its own
  const uint64_t per = align_up(layer_ws(VM_LAYER_MAX_TOKENS, K, a->inter_size, a->shared_inter, a->expert_count,
                                         a->act_dtype).total);
  const uint64_t need = per * ((T + VM_LAYER_MAX_TOKENS - 1) / VM_LAYER_MAX_TOKENS);
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)need);
  for (uint32_t t0 = 0; t0 < T; t0 += VM_LAYER_MAX_TOKENS) {
    VmLayerArgs c = *a;
    const uint32_t n = T - t0 < VM_LAYER_MAX_TOKENS ? T - t0 : VM_LAYER_MAX_TOKENS;
    c.tokens = n;
    c.workspace = static_cast<char*>(a->workspace) + per * (t0 / VM_LAYER_MAX_TOKENS);
    c.workspace_bytes = per;
    if (a->gates_out != nullptr) c.gates_out = static_cast<float*>(a->gates_out) + uint64_t(t0) * a->expert_count;
    c.x = static_cast<const float*>(a->x) + uint64_t(t0) * H;
    c.output = static_cast<float*>(a->output) + uint64_t(t0) * H;
    if (a->inds_out != nullptr) c.inds_out = a->inds_out + uint64_t(t0) * K;
    if (a->scores_out != nullptr) c.scores_out = static_cast<float*>(a->scores_out) + uint64_t(t0) * K;
    if (a->inject_out != nullptr) {
      const uint64_t streams = uint64_t(t0) * a->hc_count;
      c.inject_hidden = static_cast<const float*>(a->inject_hidden) + streams * H;
      c.inject_weights = static_cast<const float*>(a->inject_weights) + streams;
      c.inject_out = static_cast<float*>(a->inject_out) + streams * H;
    }
    rc = layer_decode(&c, stream);
    if (rc != VM_OK) return rc;
  }
  return VM_OK;
}

int vm_moe_layer_static(const VmLayerArgs* a, void* stream_ptr) {
  int rc = validate_layer(a);
  if (rc != VM_OK) return rc;
  const uint64_t need = vm_moe_layer_workspace(a->tokens, a->top_k, a->hidden_size, a->inter_size, a->shared_inter,
                                               a->expert_count, a->act_dtype);
  if (need > VM_STATIC_SCRATCH_BYTES)
    return fail(VM_EWORKSPACE, "this call needs %llu bytes of scratch, above the static %llu; call vm_moe_layer "
                "with a workspace", (unsigned long long)need, (unsigned long long)VM_STATIC_SCRATCH_BYTES);
  void* ptr = nullptr;
  rc = scratch_address(&ptr);
  if (rc != VM_OK) return rc;
  VmLayerArgs c = *a;
  c.workspace = ptr;
  c.workspace_bytes = VM_STATIC_SCRATCH_BYTES;
  t_static_call = true;
  rc = vm_moe_layer(&c, stream_ptr);
  t_static_call = false;
  return rc;
}

// Router logits (and the shared expert's sigmoid gate) of a decode call.
static hipError_t launch_layer_front(const VmLayerArgs* a, const LayerWs& w, char* ws, hipStream_t stream) {
  vm::FrontLaunch f{};
  f.x = a->x;
  f.weight = a->router_weight;
  f.bias = a->router_bias;
  f.logits = reinterpret_cast<float*>(ws + w.logits);
  if (a->shared_inter != 0) f.seg = to_ptrs(a->shared_expert_gate);
  f.shared_sig = ws + w.sig;
  f.tokens = a->tokens;
  f.hidden = a->hidden_size;
  f.experts = a->expert_count;
  f.act_dtype = static_cast<int>(a->act_dtype);
  return vm::launch_front(f, stream);
}

// The down + combine launch of a decode call: activations [T, S, I] in the
// workspace, routes as route words (slot_table null) or expert ids.
static vm::DownLaunch down_args(const VmLayerArgs* a, const LayerWs& w, char* ws, const uint32_t* routes,
                                const int32_t* slot_table, void* scores) {
  const bool shared = a->shared_inter != 0;
  vm::DownLaunch d{};
  d.act = ws + w.act;
  d.routes = routes;
  d.slot_table = slot_table;
  d.down = to_ptrs(a->down);
  if (shared) d.shared_down = to_ptrs(a->shared_down_proj);
  d.shared_sig = ws + w.sig;
  d.pool = to_pool(a->pool);
  d.scores = scores;
  d.score_dtype = static_cast<int>(a->act_dtype);
  d.out = a->output;
  d.inject = to_inject(a);
  d.generic = a->combine == VM_COMBINE_GENERIC ? 1u : 0u;
  d.status = a->status;
  d.tokens = a->tokens;
  d.slots = a->top_k;
  d.hidden = a->hidden_size;
  d.inter = a->inter_size;
  d.experts = a->expert_count;
  d.has_shared = shared ? 1 : 0;
  d.act_dtype = static_cast<int>(a->act_dtype);
  return d;
}

static int layer_decode(const VmLayerArgs* a, hipStream_t stream) {
  const uint32_t T = a->tokens, K = a->top_k, H = a->hidden_size, I = a->inter_size, E = a->expert_count;
  const bool shared = a->shared_inter != 0;
  const uint32_t S = K + (shared ? 1 : 0);
  if (!vm::gateup_supported(H)) return fail(VM_EUNSUPPORTED, "hidden_size %u is above the decode kernel bound", H);
  if (!vm::down_supported(I, S, a->act_dtype)) return fail(VM_EUNSUPPORTED, "inter_size %u is above the decode kernel bound", I);
  const LayerWs w = layer_ws(T, K, I, a->shared_inter, E, a->act_dtype);
  if (a->workspace == nullptr || a->workspace_bytes < w.total)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)w.total);
  char* ws = static_cast<char*>(a->workspace);
  int32_t* inds = a->inds_out != nullptr ? a->inds_out : reinterpret_cast<int32_t*>(ws + w.inds);
  void* scores = a->scores_out != nullptr ? a->scores_out : static_cast<void*>(ws + w.scores);
  uint32_t* words = reinterpret_cast<uint32_t*>(ws + w.words);
  float* logits = reinterpret_cast<float*>(ws + w.logits);
  const uint32_t phases = a->phases == 0 ? (VM_PHASE_ROUTER | VM_PHASE_EXPERTS) : a->phases;
  // fused: the gate/up blocks select the experts themselves from the logits;
  // split: a select kernel publishes inds/scores for the host between phases
  const bool fused = phases == (VM_PHASE_ROUTER | VM_PHASE_EXPERTS);
  hipError_t e = hipSuccess;
  vm::FusedLaunch fl{};
  uint32_t blocks = 0;
  bool two_launch = false;
  if (fused && fused_args(a, w, ws, fl, blocks, two_launch)) {
    e = vm::launch_fused_front(fl, stream);
    if (e != hipSuccess) return hip_fail(e, "router launch");
    e = vm::launch_fused_experts(fl, blocks, two_launch, stream);
    if (e != hipSuccess) return hip_fail(e, "experts launch");
    if (two_launch) return VM_OK;
    e = vm::launch_down(down_args(a, w, ws, words, nullptr, scores), stream);
    if (e != hipSuccess) return hip_fail(e, "down launch");
    return VM_OK;
  }

  if (phases & VM_PHASE_ROUTER) {
    e = launch_layer_front(a, w, ws, stream);
    if (e != hipSuccess) return hip_fail(e, "router launch");
    if (!fused) {
      vm::SelectLaunch s{};
      s.logits = logits;
      s.inds = inds;
      s.scores = scores;
      s.tokens = T;
      s.experts = E;
      s.top_k = K;
      s.act_dtype = static_cast<int>(a->act_dtype);
      s.blend = a->renorm_blend;
      s.gates = phases == VM_PHASE_ROUTER ? a->gates_out : nullptr;
      e = vm::launch_select(s, stream);
      if (e != hipSuccess) return hip_fail(e, "select launch");
    }
  }
  if (!(phases & VM_PHASE_EXPERTS)) return VM_OK;

  vm::GateUpLaunch g{};
  g.x = a->x;
  g.routes = reinterpret_cast<const uint32_t*>(inds);
  g.logits = fused ? logits : nullptr;
  g.slot_table = a->slot_table;
  g.gate = to_ptrs(a->gate);
  g.up = to_ptrs(a->up);
  if (shared) {
    g.shared_gate = to_ptrs(a->shared_gate_proj);
    g.shared_up = to_ptrs(a->shared_up_proj);
  }
  g.pool = to_pool(a->pool);
  g.act = ws + w.act;
  g.inds_out = fused ? inds : nullptr;
  g.scores_out = fused ? scores : nullptr;
  g.words_out = fused ? words : nullptr;
  g.status = a->status;
  g.tokens = T;
  g.slots = K;
  g.hidden = H;
  g.inter = I;
  g.experts = E;
  g.has_shared = shared ? 1 : 0;
  g.act_dtype = static_cast<int>(a->act_dtype);
  g.blend = a->renorm_blend;
  e = vm::launch_gateup(g, stream);
  if (e != hipSuccess) return hip_fail(e, "gate/up launch");

  e = fused ? vm::launch_down(down_args(a, w, ws, words, nullptr, scores), stream)
            : vm::launch_down(down_args(a, w, ws, reinterpret_cast<const uint32_t*>(inds), a->slot_table, scores),
                              stream);
  if (e != hipSuccess) return hip_fail(e, "down launch");
  return VM_OK;
}

// End of the last record part: the bytes of a record a fill copies.
static uint64_t record_end(const VmPoolView& v, uint32_t hidden, uint32_t inter) {
  const uint64_t w = uint64_t(inter) * hidden / 2, m = uint64_t(inter) * (hidden / 32) * 2;
  const uint64_t dm = uint64_t(hidden) * (inter / 32) * 2;
  const uint64_t sizes[VM_PARTS] = {w, m, m, w, m, m, w, dm, dm};
  uint64_t end = 0;
  for (int i = 0; i < VM_PARTS; ++i) end = v.part_offset[i] + sizes[i] > end ? v.part_offset[i] + sizes[i] : end;
  return end;
}

// Device-accessible address of pinned host memory (cached for the last store).
static int host_device_pointer(const void* host, const uint8_t** out) {
  thread_local const void* last_host = nullptr;
  thread_local const uint8_t* last_dev = nullptr;
  if (host != last_host) {
    void* dev = nullptr;
    hipError_t e = hipHostGetDevicePointer(&dev, const_cast<void*>(host), 0);
    if (e != hipSuccess || dev == nullptr)
      return fail(VM_EINVAL, "host_store is not pinned host memory (hipHostGetDevicePointer: %s)",
                  hipGetErrorString(e));
    last_host = host;
    last_dev = static_cast<const uint8_t*>(dev);
  }
  *out = last_dev;
  return VM_OK;
}

// Workspace of vm_hyper_mix: normed [T, n] then d [T, lowrank], activation dtype.
static uint64_t hyper_normed_bytes(uint32_t tokens, uint32_t n, uint32_t act_dtype) {
  return align_up(uint64_t(tokens) * n * (act_dtype == VM_F32 ? 4 : 2));
}

uint64_t vm_hyper_mix_workspace(uint32_t tokens, uint32_t hc_count, uint32_t hidden_size, uint32_t lowrank,
                                uint32_t act_dtype) {
  const uint32_t n = hc_count * hidden_size;
  return hyper_normed_bytes(tokens, n, act_dtype) + align_up(uint64_t(tokens) * lowrank * (act_dtype == VM_F32 ? 4 : 2));
}

int vm_hyper_mix(const VmHyperArgs* a, void* stream_ptr) {
  if (a == nullptr) return fail(VM_EINVAL, "null arguments");
  const uint32_t T = a->tokens, H = a->hidden_size, hc = a->hc_count, r = a->lowrank;
  if (T == 0 || H == 0) return fail(VM_EINVAL, "tokens and hidden_size must be positive");
  if (T > 65535) return fail(VM_EUNSUPPORTED, "at most 65535 tokens per call");
  if (hc == 0 || hc > VM_MAX_STREAMS) return fail(VM_EINVAL, "hc_count must be 1..%d", VM_MAX_STREAMS);
  if (a->act_dtype != VM_BF16 && a->act_dtype != VM_F32) return fail(VM_EINVAL, "act_dtype must be bf16 or f32");
  const uint64_t n64 = uint64_t(hc) * H;
  if (n64 % 64 || n64 > vm::kHcMaxRow)
    return fail(VM_EUNSUPPORTED, "hc_count * hidden_size must be a multiple of 64 up to %u", vm::kHcMaxRow);
  const uint32_t n = static_cast<uint32_t>(n64);
  if (r == 0 || r % 32 || r > vm::kHcMaxLowrank)
    return fail(VM_EUNSUPPORTED, "lowrank must be a multiple of 32 up to %u", vm::kHcMaxLowrank);
  const uint32_t gs = a->norm_group == 0 ? n : a->norm_group;
  if (gs % 64 || n % gs) return fail(VM_EUNSUPPORTED, "norm_group must be 0 or a multiple of 64 dividing the row");
  if (a->hidden == nullptr || a->norm_weight == nullptr || a->mixed == nullptr || a->weights == nullptr)
    return fail(VM_EINVAL, "hidden, norm_weight, mixed and weights are required");
  if (!aligned16(a->hidden)) return fail(VM_EINVAL, "hidden must be 16-byte aligned");
  if (a->mix_down.weight == nullptr || a->mix_up.weight == nullptr || a->inject.weight == nullptr ||
      !proj_ok(a->mix_down) || !proj_ok(a->mix_up) || !proj_ok(a->inject))
    return fail(VM_EINVAL, "mix_down, mix_up and inject projections are required");
  if (!aligned16(a->mix_down.weight) || !aligned16(a->mix_up.weight) || !aligned16(a->inject.weight))
    return fail(VM_EINVAL, "projection weights must be 16-byte aligned");
  const uint64_t need = vm_hyper_mix_workspace(T, hc, H, r, a->act_dtype);
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)need);
  char* ws = static_cast<char*>(a->workspace);
  vm::HcLaunch p{};
  p.hidden = a->hidden;
  p.norm_weight = a->norm_weight;
  p.down = to_ptrs(a->mix_down);
  p.up = to_ptrs(a->mix_up);
  p.inj = to_ptrs(a->inject);
  p.normed = a->normed != nullptr ? a->normed : ws;
  p.d = ws + hyper_normed_bytes(T, n, a->act_dtype);
  p.mixed = a->mixed;
  p.weights = a->weights;
  p.eps = a->eps;
  p.tokens = T;
  p.width = H;
  p.hc = hc;
  p.n = n;
  p.lowrank = r;
  p.norm_group = gs;
  p.one_centered = a->one_centered ? 1u : 0u;
  p.act_dtype = static_cast<int>(a->act_dtype);
  const hipError_t e = vm::launch_hyper_mix(p, static_cast<hipStream_t>(stream_ptr));
  if (e != hipSuccess) return hip_fail(e, "hyper-connection launch");
  return VM_OK;
}

int vm_moe_layer_lru(const VmLayerArgs* a, const VmDeviceLru* lru, void* stream_ptr) {
  if (a == nullptr || lru == nullptr) return fail(VM_EINVAL, "null arguments");
  const hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const uint32_t T = a->tokens, K = a->top_k, H = a->hidden_size, I = a->inter_size, E = a->expert_count;
  if (T == 0 || T > VM_LAYER_MAX_TOKENS)
    return fail(VM_EUNSUPPORTED, "the device LRU serves decode calls of 1..%d tokens", VM_LAYER_MAX_TOKENS);
  if (a->phases != 0) return fail(VM_EINVAL, "vm_moe_layer_lru runs the whole layer (phases must be 0)");
  if (lru->slot_table == nullptr || lru->slot_owner == nullptr || lru->lru_order == nullptr ||
      lru->counters == nullptr || lru->host_row == nullptr || lru->host_store == nullptr)
    return fail(VM_EINVAL, "device LRU state pointers are required");
  if (a->pool.base == nullptr) return fail(VM_EINVAL, "the device LRU needs a pool view");
  if (lru->layer >= lru->layers) return fail(VM_EINVAL, "layer %u is outside 0..%u", lru->layer, lru->layers);
  if (lru->slots != a->pool.records)
    return fail(VM_EINVAL, "LRU slots (%u) must equal the pool records (%u)", lru->slots, a->pool.records);
  if (lru->slots > vm::kLruMaxSlots)
    return fail(VM_EUNSUPPORTED, "the device LRU holds at most %u slots", vm::kLruMaxSlots);
  if (lru->order_len > lru->slots)
    return fail(VM_EINVAL, "order_len (%u) exceeds the slots (%u)", lru->order_len, lru->slots);
  if (uint64_t(T) * K > lru->order_len || uint64_t(T) * K > vm::kLruMaxRouted)
    return fail(VM_EINVAL, "tokens * top_k = %u exceeds the queued slots or the %u routed ids of one call", T * K,
                vm::kLruMaxRouted);
  if (uint64_t(lru->layers) * E > 0x7fffffffull) return fail(VM_EINVAL, "layers * expert_count is too large");
  VmLayerArgs r = *a;
  r.slot_table = lru->slot_table + uint64_t(lru->layer) * E;
  int rc = validate_layer(&r);
  if (rc != VM_OK) return rc;
  const uint64_t bytes = record_end(a->pool, H, I);
  if (bytes % 16 || lru->host_stride % 16 || lru->host_stride < bytes || a->pool.header_size % 16 ||
      bytes / 16 * vm::kLruMaxRouted >= (1ull << 32))
    return fail(VM_EINVAL, "records of %llu bytes need 16-byte aligned host rows of at least that size",
                (unsigned long long)bytes);
  if (!aligned16(lru->host_store)) return fail(VM_EINVAL, "host_store must be 16-byte aligned");
  const uint8_t* host = nullptr;
  rc = host_device_pointer(lru->host_store, &host);
  if (rc != VM_OK) return rc;
  const LayerWs w = layer_ws(T, K, I, a->shared_inter, E, a->act_dtype);
  if (a->workspace == nullptr || a->workspace_bytes < w.total)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)w.total);
  char* ws = static_cast<char*>(a->workspace);

  // 1. router logits and shared gate (with the one-token pipeline: also the
  //    shared expert's gate/up)
  vm::FusedLaunch fl{};
  uint32_t blocks = 0;
  bool two_launch = false;
  const bool one_token = fused_args(&r, w, ws, fl, blocks, two_launch);
  hipError_t e = one_token ? vm::launch_fused_front(fl, stream) : launch_layer_front(a, w, ws, stream);
  if (e != hipSuccess) return hip_fail(e, "router launch");
  // 2. softmax/top-k into inds/scores and assign() on the device state, one block
  int32_t* inds = a->inds_out != nullptr ? a->inds_out : reinterpret_cast<int32_t*>(ws + w.inds);
  vm::SelectLaunch sel{};
  sel.logits = reinterpret_cast<const float*>(ws + w.logits);
  sel.inds = inds;
  sel.scores = a->scores_out != nullptr ? a->scores_out : static_cast<void*>(ws + w.scores);
  sel.tokens = T;
  sel.experts = E;
  sel.top_k = K;
  sel.act_dtype = static_cast<int>(a->act_dtype);
  sel.blend = a->renorm_blend;
  uint32_t* fill = reinterpret_cast<uint32_t*>(ws + w.fill);
  vm::LruLaunch l{};
  l.slot_table = lru->slot_table;
  l.slot_owner = lru->slot_owner;
  l.lru_order = lru->lru_order;
  l.counters = lru->counters;
  l.host_row = lru->host_row;
  l.fill_count = fill;
  l.fill_src = fill + 1;
  l.fill_dst = fill + 1 + vm::kLruMaxRouted;
  l.status = a->status;
  l.host_records = lru->host_records;
  l.routed = T * K;
  l.experts = E;
  l.layers = lru->layers;
  l.layer = lru->layer;
  l.slots = lru->slots;
  l.order_len = lru->order_len;
  e = vm::launch_select_lru(sel, l, stream);
  if (e != hipSuccess) return hip_fail(e, "select/lru launch");
  vm::FillLaunch f{};
  f.count = l.fill_count;
  f.src = l.fill_src;
  f.dst = l.fill_dst;
  f.host = host;
  f.host_stride = lru->host_stride;
  f.host_records = lru->host_records;
  f.pool = const_cast<uint8_t*>(a->pool.base);
  f.header = a->pool.header_size;
  f.stride = a->pool.record_stride;
  f.pool_records = a->pool.records;
  f.record_bytes = bytes;
  e = vm::launch_fill(f, stream);
  if (e != hipSuccess) return hip_fail(e, "fill launch");
  // 4. the experts through the updated slot table
  if (one_token) {
    fl.routes = inds;
    fl.route_scores = static_cast<const uint16_t*>(sel.scores);
    fl.inds_out = nullptr;
    fl.scores_out = nullptr;
    e = vm::launch_fused_experts(fl, blocks, two_launch, stream);
    if (e != hipSuccess) return hip_fail(e, "experts launch");
    if (two_launch) return VM_OK;
    e = vm::launch_down(down_args(&r, w, ws, fl.words_out, nullptr, sel.scores), stream);
    if (e != hipSuccess) return hip_fail(e, "down launch");
    return VM_OK;
  }
  r.phases = VM_PHASE_EXPERTS;
  return layer_decode(&r, stream);
}


// The experts of the grouped path: sort the routes, gate/up + SwiGLU and down
// over every group's rows, combine.  `sig`/shared projections are used when
// `shared` is set (the layer's own shared expert).
struct GroupedExperts {
  const void* x;
  const int32_t* inds;
  const void* scores;
  VmQ4Proj gate, up, down;
  VmPoolView pool;
  const int32_t* slot_table;
  bool shared;
  VmQ4Proj shared_gate, shared_up, shared_down;
  const void* sig;
  const void* shared_y;
  // the shared expert ran on the side stream: its output rows, and the event
  // the combine waits for (shared is then false for the sort and the GEMMs)
  const uint16_t* shared_rows;
  hipEvent_t shared_join;
  void* output;
  vm::Inject inject;
  uint32_t* status;
  uint32_t T, K, H, I, E;
  int mode;
  bool counted;  // the sort's counters were zeroed by the router GEMM
};

static int run_grouped_experts(const GroupedExperts& g, const GroupedWs& w, char* ws, hipStream_t stream) {
  // the chunked GEMM addresses its activation matrices with 32-bit byte
  // offsets and its outputs with 32-bit element indices
  const uint64_t sorted_rows = uint64_t(g.T) * g.K + g.T;
  if (uint64_t(g.T) * g.H * 2 > 0xffffffffull || sorted_rows * g.I * 2 > 0xffffffffull ||
      sorted_rows * g.H > 0xffffffffull)
    return fail(VM_EUNSUPPORTED, "grouped call of %u tokens: an activation matrix of 4 GiB or more", g.T);
  vm::SortLaunch s{};
  s.inds = g.inds;
  s.row_off = reinterpret_cast<uint32_t*>(ws + w.row_off);
  s.tiles = reinterpret_cast<uint2*>(ws + w.tiles);
  s.tile_count = reinterpret_cast<uint32_t*>(ws + w.tile_count);
  s.tiles_dn = reinterpret_cast<uint2*>(ws + w.tiles_dn);
  s.tile_count_dn = reinterpret_cast<uint32_t*>(ws + w.tile_count_dn);
  s.counts = reinterpret_cast<uint32_t*>(ws + w.sort_counts);
  s.cursors = reinterpret_cast<uint32_t*>(ws + w.sort_cursors);
  s.row_token = reinterpret_cast<uint32_t*>(ws + w.row_token);
  s.pair_row = reinterpret_cast<uint32_t*>(ws + w.pair_row);
  s.status = g.status;
  s.tokens = g.T;
  s.slots = g.K;
  s.experts = g.E;
  s.shared_rows = g.shared ? g.T : 0;
  s.tile_rows = w.tile_rows;
  s.tile_rows_dn = w.tile_rows_dn;
  hipError_t e = g.counted ? vm::launch_sort_counted(s, stream) : vm::launch_sort(s, stream);
  if (e != hipSuccess) return hip_fail(e, "sort launch");

  vm::GroupedLaunch q{};
  q.row_off = s.row_off;
  q.tiles = s.tiles;
  q.tile_count = s.tile_count;
  q.slot_table = g.slot_table;
  q.pool = to_pool(g.pool);
  q.status = g.status;
  q.experts = g.E;
  // gate/up + SwiGLU over the gathered token rows
  q.a = static_cast<const uint16_t*>(g.x);
  q.row_token = s.row_token;
  q.dense[0] = to_ptrs(g.gate);
  q.dense[1] = to_ptrs(g.up);
  if (g.shared) {
    q.shared[0] = to_ptrs(g.shared_gate);
    q.shared[1] = to_ptrs(g.shared_up);
  }
  q.part[0] = 0;
  q.part[1] = 1;
  q.out = ws + w.act;
  q.k_dim = g.H;
  q.n_dim = g.I;
  q.a_stride = g.H;
  q.a_rows = g.T;
  // routed rows per expert on average: at most one row tile each
  // (the tall instance loads its weights through the caches: an expert's
  // tiles, and its gate and up halves' column slices, share them)
  q.weights_once = uint64_t(g.T) * g.K <= uint64_t(g.E) * w.tile_rows && w.tile_rows != vm::kGroupedRowsTall;
  q.tile_rows = w.small ? 0u : w.tile_rows;
  e = w.small ? vm::launch_rows(vm::kEpiSwiglu, q, w.max_tiles, stream)
              : vm::launch_grouped(vm::kEpiSwiglu, q, w.max_tiles, stream);
  if (e != hipSuccess) return hip_fail(e, "grouped gate/up launch");
  // down over the contiguous activation rows
  q.a = reinterpret_cast<const uint16_t*>(ws + w.act);
  q.row_token = nullptr;
  q.dense[0] = to_ptrs(g.down);
  q.dense[1] = vm::ProjPtrs{};
  q.shared[0] = g.shared ? to_ptrs(g.shared_down) : vm::ProjPtrs{};
  q.shared[1] = vm::ProjPtrs{};
  q.part[0] = 2;
  q.out = ws + w.rows;
  q.k_dim = g.I;
  q.n_dim = g.H;
  q.a_stride = g.I;
  q.a_rows = g.T * g.K + (g.shared ? g.T : 0);
  q.weights_once = uint64_t(g.T) * g.K <= uint64_t(g.E) * vm::kGroupedRowsDown;
  q.tile_rows = w.small || w.tile_rows_dn == vm::kGroupedRowsDown ? 0u : w.tile_rows_dn;
  q.tiles = s.tiles_dn;
  q.tile_count = s.tile_count_dn;
  e = w.small ? vm::launch_rows(vm::kEpiRows, q, w.max_tiles_dn, stream)
              : vm::launch_grouped(vm::kEpiRows, q, w.max_tiles_dn, stream);
  if (e != hipSuccess) return hip_fail(e, "grouped down launch");

  vm::CombineLaunch c{};
  c.rows = reinterpret_cast<const uint16_t*>(ws + w.rows);
  c.pair_row = s.pair_row;
  c.scores = g.scores;
  c.score_dtype = VM_BF16;
  if (g.shared) {
    c.shared_first = s.row_off + g.E;
    c.shared_sig = g.sig;
  } else if (g.shared_rows != nullptr) {
    c.shared_rows = g.shared_rows;
    c.shared_sig = g.sig;
    e = hipStreamWaitEvent(stream, g.shared_join, 0);
    if (e != hipSuccess) return hip_fail(e, "join of the shared expert's stream");
  }
  c.shared_y = g.shared_y;
  c.out = g.output;
  c.inject = g.inject;
  c.tokens = g.T;
  c.slots = g.K;
  c.hidden = g.H;
  c.mode = g.mode;
  e = vm::launch_grouped_combine(c, stream);
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return VM_OK;
}

// The shared expert of a grouped call over all T rows, with no sort: its
// sigmoid gate into sig, gate/up + SwiGLU into sh_act [T, I] and down into
// sh_rows [T, H] (one-group launches of the chunked GEMM).
static hipError_t launch_shared_expert(const VmLayerArgs* a, uint16_t* sig, uint16_t* sh_act, uint16_t* sh_rows,
                                       hipStream_t stream) {
  const uint32_t T = a->tokens, H = a->hidden_size, I = a->inter_size;
  hipError_t e = vm::launch_shared_gate(static_cast<const uint16_t*>(a->x), to_ptrs(a->shared_expert_gate), sig, T,
                                        H, stream);
  if (e != hipSuccess) return e;
  vm::GroupedLaunch q{};
  q.a = static_cast<const uint16_t*>(a->x);
  q.rows = T;
  q.experts = 0;  // every tile is the shared expert's
  q.shared[0] = to_ptrs(a->shared_gate_proj);
  q.shared[1] = to_ptrs(a->shared_up_proj);
  q.part[0] = 0;
  q.part[1] = 1;
  q.out = sh_act;
  q.status = a->status;
  q.k_dim = H;
  q.n_dim = I;
  q.a_stride = H;
  q.a_rows = T;
  // the same tile height as the call's routed gate/up (tall tiles by the
  // shared expert's own T rows measured no faster)
  const uint32_t tr = gateup_tile_rows(T, a->top_k, H, a->expert_count);
  q.tile_rows = tr == vm::kGroupedRows ? 0u : tr;
  e = vm::launch_grouped(vm::kEpiSwiglu, q, (T + tr - 1) / tr, stream);
  if (e != hipSuccess) return e;
  q.a = sh_act;
  // its own group of T rows: tall tiles above 48 rows (each
  // weight dequantised half as often, which leaves the routed gate/up it runs
  // beside more of the CUs)
  const uint32_t trd = down_tile_rows(T, 1, I, 1);
  q.tile_rows = trd == vm::kGroupedRowsDown ? 0u : trd;
  q.shared[0] = to_ptrs(a->shared_down_proj);
  q.shared[1] = vm::ProjPtrs{};
  q.part[0] = 2;
  q.out = sh_rows;
  q.k_dim = I;
  q.n_dim = H;
  q.a_stride = I;
  return vm::launch_grouped(vm::kEpiRows, q, (T + trd - 1) / trd, stream);
}

static int layer_grouped(const VmLayerArgs* a, hipStream_t stream) {
  const uint32_t T = a->tokens, K = a->top_k, H = a->hidden_size, I = a->inter_size, E = a->expert_count;
  const bool shared = a->shared_inter != 0;
  const GroupedWs w = grouped_ws(T, K, H, I, E, shared);
  if (a->workspace == nullptr || a->workspace_bytes < w.total)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)w.total);
  if (!aligned16(a->output)) return fail(VM_EINVAL, "output must be 16-byte aligned");
  char* ws = static_cast<char*>(a->workspace);
  int32_t* inds = a->inds_out != nullptr ? a->inds_out : reinterpret_cast<int32_t*>(ws + w.inds);
  void* scores = a->scores_out != nullptr ? a->scores_out : static_cast<void*>(ws + w.scores);
  uint16_t* sig = reinterpret_cast<uint16_t*>(ws + w.sig);
  const uint32_t phases = a->phases == 0 ? (VM_PHASE_ROUTER | VM_PHASE_EXPERTS) : a->phases;
  hipError_t e = hipSuccess;
  // Calls above the one-block sort's size that run the router GEMM and the
  // experts together: the GEMM zeroes the sort's counters, so the sort is a
  // count and one layout + scatter launch.
  const bool counted = T > kFrontMaxTokens && uint64_t(T) * K > vm::kSortOneBlockPairs &&
                       (phases & VM_PHASE_ROUTER) && (phases & VM_PHASE_EXPERTS);
  // Calls above kSideMinTokens rows run the shared expert on the side stream,
  // into the last T rows of the activation and expert-row buffers (the routed
  // rows take at most the first T * K).
  SideStream* side = nullptr;
  if (shared && T > kSideMinTokens && (phases & VM_PHASE_ROUTER) && (phases & VM_PHASE_EXPERTS))
    side = side_stream(stream);
  uint16_t* sh_rows = reinterpret_cast<uint16_t*>(ws + w.rows) + uint64_t(T) * K * H;
  if (side != nullptr) {
    e = hipEventRecord(side->fork, stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(side->stream, side->fork, 0);
    if (e != hipSuccess) return hip_fail(e, "fork of the shared expert's stream");
    e = launch_shared_expert(a, sig, reinterpret_cast<uint16_t*>(ws + w.act) + uint64_t(T) * K * I, sh_rows,
                             side->stream);
    const hipError_t j = hipEventRecord(side->join, side->stream);
    if (e != hipSuccess || j != hipSuccess) {
      if (j == hipSuccess) (void)hipStreamWaitEvent(stream, side->join, 0);
      return hip_fail(e != hipSuccess ? e : j, "shared expert launch");
    }
  }
  // a failure after the fork still joins the side stream (a capture must not
  // end with it forked); on success the combine has joined it
  auto done = [&](int rc) {
    if (side != nullptr && rc != VM_OK) (void)hipStreamWaitEvent(stream, side->join, 0);
    return rc;
  };
  if ((phases & VM_PHASE_ROUTER) && T <= kFrontMaxTokens) {
    // few rows: the decode router (one row per wave, every token) and shared gate
    vm::FrontLaunch f{};
    f.x = a->x;
    f.weight = a->router_weight;
    f.bias = a->router_bias;
    f.logits = reinterpret_cast<float*>(ws + w.logits);
    if (shared) f.seg = to_ptrs(a->shared_expert_gate);
    f.shared_sig = sig;
    f.tokens = T;
    f.hidden = H;
    f.experts = E;
    f.act_dtype = VM_BF16;
    e = vm::launch_front(f, stream);
    if (e != hipSuccess) return done(hip_fail(e, "router launch"));
  } else if (phases & VM_PHASE_ROUTER) {
    // router logits as an MFMA GEMM over all rows (32-bit output indices)
    if (uint64_t(T) * E > 0xffffffffull || uint64_t(T) * H * 2 > 0xffffffffull)
      return done(fail(VM_EUNSUPPORTED, "grouped call of %u tokens: the router GEMM's matrices are too large", T));
    vm::GroupedLaunch r{};
    r.a = static_cast<const uint16_t*>(a->x);
    r.rows = T;
    r.bf16_weight = a->router_weight;
    r.bias = a->router_bias;
    r.out = ws + w.logits;
    r.k_dim = H;
    r.n_dim = E;
    r.a_stride = H;
    r.a_rows = T;
    r.experts = E;
    if (counted) {
      r.zero_words = reinterpret_cast<uint32_t*>(ws + w.sort_counts);
      r.zero_count = 2048;
    }
    e = VM_ROUTER_RING && vm::router_gemm_supported(H, E)
            ? vm::launch_router_gemm(r, stream)
            : vm::launch_grouped(vm::kEpiLogits, r, (T + vm::kGroupedRowsRouter - 1) / vm::kGroupedRowsRouter, stream);
    if (e != hipSuccess) return done(hip_fail(e, "router launch"));
  }
  if (phases & VM_PHASE_ROUTER) {
    // softmax / top-k / renorm per row
    vm::SelectLaunch s{};
    s.logits = reinterpret_cast<const float*>(ws + w.logits);
    s.inds = inds;
    s.scores = scores;
    s.tokens = T;
    s.experts = E;
    s.top_k = K;
    s.act_dtype = VM_BF16;
    s.blend = a->renorm_blend;
    s.gates = phases == VM_PHASE_ROUTER ? a->gates_out : nullptr;
    if (shared && side == nullptr && T > kFrontMaxTokens) {
      // the shared expert as a sorted group: its sigmoid gate by the selection's waves
      s.gate_x = static_cast<const uint16_t*>(a->x);
      s.seg = to_ptrs(a->shared_expert_gate);
      s.shared_sig = sig;
      s.hidden = H;
    }
    e = vm::launch_select(s, stream);
    if (e != hipSuccess) return done(hip_fail(e, "select launch"));
  }
  if (!(phases & VM_PHASE_EXPERTS)) return VM_OK;
  GroupedExperts g{};
  g.x = a->x;
  g.inds = inds;
  g.scores = scores;
  g.gate = a->gate;
  g.up = a->up;
  g.down = a->down;
  g.pool = a->pool;
  g.slot_table = a->slot_table;
  g.shared = shared && side == nullptr;
  g.shared_gate = a->shared_gate_proj;
  g.shared_up = a->shared_up_proj;
  g.shared_down = a->shared_down_proj;
  g.sig = sig;
  if (side != nullptr) {
    g.shared_rows = sh_rows;
    g.shared_join = side->join;
  }
  g.output = a->output;
  g.inject = to_inject(a);
  g.status = a->status;
  g.T = T;
  g.K = K;
  g.H = H;
  g.I = I;
  g.E = E;
  g.mode = 1;  // rows > 8: the reference's generic combine
  g.counted = counted;
  return done(run_grouped_experts(g, w, ws, stream));
}

uint64_t vm_moe_grouped_workspace(uint32_t tokens, uint32_t top_k, uint32_t hidden_size, uint32_t inter_size,
                                  uint32_t expert_count, uint32_t act_dtype) {
  (void)act_dtype;
  return grouped_ws(tokens, top_k, hidden_size, inter_size, expert_count, false).total;
}

int vm_moe_grouped(const VmGroupedArgs* a, void* stream_ptr) {
  if (a == nullptr) return fail(VM_EINVAL, "null arguments");
  const uint32_t T = a->tokens, K = a->top_k, H = a->hidden_size, I = a->inter_size, E = a->expert_count;
  if (a->act_dtype != VM_BF16) return fail(VM_EUNSUPPORTED, "the grouped kernels take bf16 activations");
  if (T == 0 || K == 0 || K > kMaxTopK) return fail(VM_EINVAL, "tokens must be positive and top_k in 1..%u", kMaxTopK);
  if (E == 0 || E > kMaxExperts) return fail(VM_EINVAL, "expert_count must be in 1..%u", kMaxExperts);
  if (H == 0 || H % 32 || I == 0 || I % 32) return fail(VM_EINVAL, "hidden_size and inter_size must be multiples of 32");
  if (a->group_size != 32) return fail(VM_EUNSUPPORTED, "group_size must be 32");
  if (a->combine_mode > 2) return fail(VM_EINVAL, "combine_mode must be 0, 1 or 2");
  if (a->x == nullptr || a->inds == nullptr || a->output == nullptr)
    return fail(VM_EINVAL, "x, inds and output are required");
  if (a->combine_mode != 2 && a->scores == nullptr) return fail(VM_EINVAL, "scores are required to combine");
  if (!aligned16(a->x) || !aligned16(a->output) || (a->shared_y != nullptr && !aligned16(a->shared_y)))
    return fail(VM_EINVAL, "x, output and shared_y must be 16-byte aligned");
  if (a->slot_table != nullptr && a->pool.base == nullptr) return fail(VM_EINVAL, "a slot table needs a pool view");
  if (a->slot_table == nullptr && a->gate.weight == nullptr && a->pool.base == nullptr)
    return fail(VM_EINVAL, "experts need a slot table with a pool view, or dense projections");
  if (!proj_ok(a->gate) || !proj_ok(a->up) || !proj_ok(a->down)) return fail(VM_EINVAL, "malformed projection");
  int rc = check_pool(a->pool, H, I);
  if (rc != VM_OK) return rc;
  const GroupedWs w = grouped_ws(T, K, H, I, E, false);
  if (a->workspace == nullptr || a->workspace_bytes < w.total)
    return fail(VM_EWORKSPACE, "workspace of %llu bytes needed", (unsigned long long)w.total);
  GroupedExperts g{};
  g.x = a->x;
  g.inds = a->inds;
  g.scores = a->scores;
  g.gate = a->gate;
  g.up = a->up;
  g.down = a->down;
  g.pool = a->pool;
  g.slot_table = a->slot_table;
  g.shared_y = a->shared_y;
  g.output = a->output;
  g.status = a->status;
  g.T = T;
  g.K = K;
  g.H = H;
  g.I = I;
  g.E = E;
  g.mode = static_cast<int>(a->combine_mode);
  return run_grouped_experts(g, w, static_cast<char*>(a->workspace), static_cast<hipStream_t>(stream_ptr));
}

// ------------------------------------------------------------ combine ---

int vm_weighted_combine(const void* expert_outputs, const void* scores, void* out, uint32_t tokens, uint32_t slots,
                        uint32_t hidden_size, uint32_t act_dtype, uint32_t score_dtype, void* stream) {
  if (expert_outputs == nullptr || scores == nullptr || out == nullptr) return fail(VM_EINVAL, "null pointer");
  if (act_dtype > VM_F32 || score_dtype > VM_F32) return fail(VM_EINVAL, "unknown dtype");
  if (tokens == 0 || slots == 0 || hidden_size == 0) return fail(VM_EINVAL, "empty combine");
  hipError_t e = vm::launch_weighted_combine(expert_outputs, scores, out, tokens, slots, hidden_size,
                                             static_cast<int>(act_dtype), static_cast<int>(score_dtype),
                                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return VM_OK;
}

// -------------------------------------------------------------- stage ---

int vm_pool_stage(void* pool_base, uint64_t header_size, uint64_t record_stride, uint64_t pool_records,
                  const void* src_host, uint64_t src_stride, uint64_t src_records, uint64_t record_bytes,
                  const int64_t* src_index, const int64_t* dst_slot, uint32_t count, void* stream) {
  if (count == 0) return VM_OK;
  if (pool_base == nullptr || src_host == nullptr || src_index == nullptr || dst_slot == nullptr)
    return fail(VM_EINVAL, "null pointer");
  if (record_bytes == 0 || record_bytes > record_stride || record_bytes > src_stride)
    return fail(VM_EINVAL, "record_bytes must be in 1..min(record_stride, src_stride)");
  for (uint32_t i = 0; i < count; ++i) {
    if (src_index[i] < 0 || uint64_t(src_index[i]) >= src_records)
      return fail(VM_EINVAL, "src_index[%u] = %lld is outside 0..%llu", i, (long long)src_index[i],
                  (unsigned long long)src_records);
    if (dst_slot[i] < 0 || uint64_t(dst_slot[i]) >= pool_records)
      return fail(VM_EINVAL, "dst_slot[%u] = %lld is outside 0..%llu", i, (long long)dst_slot[i],
                  (unsigned long long)pool_records);
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t i = 0;
  while (i < count) {
    uint32_t j = i + 1;
    // merge runs that are consecutive on both sides when the strides agree
    while (j < count && record_bytes == record_stride && record_stride == src_stride &&
           src_index[j] == src_index[i] + (j - i) && dst_slot[j] == dst_slot[i] + (j - i))
      ++j;
    const uint64_t bytes = (j - i - 1) * record_stride + record_bytes;
    char* dst = static_cast<char*>(pool_base) + header_size + uint64_t(dst_slot[i]) * record_stride;
    const char* src = static_cast<const char*>(src_host) + uint64_t(src_index[i]) * src_stride;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
    i = j;
  }
  return VM_OK;
}

// ------------------------------------------------------------- timing ---

int vm_decode_pipeline(int mode) {
  if (mode < -1 || mode > 2) return fail(VM_EINVAL, "mode must be -1 (query) or 0..2");
  if (!VM_FUSED_PIPELINES && mode > 0)
    return fail(VM_EUNSUPPORTED, "pipelines 1 and 2 are built only with -DVM_FUSED_PIPELINES=1");
  if (mode == -1) return g_fused_decode.load();
  return g_fused_decode.exchange(mode);
}

int vm_timing_enable(int enabled) {
  Timing& t = timing();
  std::lock_guard<std::mutex> lock(t.mu);
  t.enabled = enabled != 0;
  return VM_OK;
}

int vm_timing_read(const char* name, double* total_ms, uint64_t* launches) {
  if (name == nullptr || total_ms == nullptr || launches == nullptr) return fail(VM_EINVAL, "null pointer");
  Timing& t = timing();
  std::lock_guard<std::mutex> lock(t.mu);
  int rc = drain_timing(t);
  if (rc != VM_OK) return rc;
  auto it = t.totals.find(name);
  *total_ms = it == t.totals.end() ? 0.0 : it->second.first;
  *launches = it == t.totals.end() ? 0 : it->second.second;
  return VM_OK;
}

int vm_timing_reset(void) {
  Timing& t = timing();
  std::lock_guard<std::mutex> lock(t.mu);
  int rc = drain_timing(t);
  t.totals.clear();
  return rc;
}

// ------------------------------------------------------------- trace ----

static struct {
  std::mutex mu;
  uint64_t* buf = nullptr;
  uint64_t capacity = 0;  // records of 8 uint64
  uint64_t used = 0;
} g_trace;

int vm_trace_set(void* device_buffer, uint64_t bytes) {
  std::lock_guard<std::mutex> lock(g_trace.mu);
  g_trace.buf = static_cast<uint64_t*>(device_buffer);
  g_trace.capacity = device_buffer != nullptr ? bytes / (8 * vm::kTraceWords) : 0;
  g_trace.used = 0;
  return VM_OK;
}

uint64_t vm_trace_records(void) {
  std::lock_guard<std::mutex> lock(g_trace.mu);
  return g_trace.used;
}

}  // extern "C"

namespace vm {

uint64_t* trace_reserve(uint32_t blocks) {
  std::lock_guard<std::mutex> lock(g_trace.mu);
  if (g_trace.buf == nullptr || g_trace.used + blocks > g_trace.capacity) return nullptr;
  uint64_t* p = g_trace.buf + g_trace.used * kTraceWords;
  g_trace.used += blocks;
  return p;
}

}  // namespace vm

extern "C" {

// The grouped (prefill / batched) path lives in grouped.hip.

}  // extern "C"
