// Host-side launch parameters shared between the C ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vm_common.h"

namespace vm {

// Route word written for a selected expert that has no pool slot: it is not
// a slot word and is above every dense expert index, so resolution fails and
// the status flag is raised.
constexpr uint32_t kMissWord = 0x7fffffffu;

// K1: router logits (and the shared expert's sigmoid gate).
struct FrontLaunch {
  const void* x;               // [T, H]
  const uint16_t* weight;      // [E, H] bf16
  const float* bias;           // optional [E]
  float* logits;               // [T, E], rounded to the activation type
  ProjPtrs seg;                // optional shared expert gate (H -> 1 Q4 row)
  void* shared_sig;            // [T] activation dtype
  uint64_t* trace;             // optional phase timestamps, 8 per block
  uint32_t tokens, hidden, experts;
  int act_dtype;
};

// Softmax / top-k / renormalisation of logits, one wave per token.
struct SelectLaunch {
  const float* logits;         // [T, E]
  int32_t* inds;               // [T, K]
  void* scores;                // [T, K] activation dtype
  void* gates;                 // optional [T, E]
  uint32_t tokens, experts, top_k;
  int act_dtype;
  float blend;
  // optional (bf16 grouped calls whose shared expert is a sorted group): the
  // shared expert's sigmoid gate of each token, computed by the same wave
  const uint16_t* gate_x;      // [T, hidden]
  ProjPtrs seg;                // H -> 1 Q4 gate row; seg.w null: none
  uint16_t* shared_sig;        // [T]
  uint32_t hidden;
};

// K2: gate/up + SwiGLU of every (token, slot) pair and the shared pairs.
struct GateUpLaunch {
  const void* x;               // [T, H]
  const uint32_t* routes;      // [T, K] route words (or expert ids with slot_table) when logits == null
  const float* logits;         // [T, E]: select the experts in the block prologue instead
  const int32_t* slot_table;   // optional expert -> slot
  ProjPtrs gate, up;           // dense routed experts
  ProjPtrs shared_gate, shared_up;  // dense shared expert (pair j == K), optional
  PoolDev pool;
  PoolDev stream;              // records for routes without the slot bit, optional
  void* act;                   // [T, S, I], S = K + has_shared
  void* gate_out;              // optional [T, K, I]
  void* up_out;                // optional [T, K, I]
  int32_t* inds_out;           // logits path: [T, K] selected experts
  void* scores_out;            // logits path: [T, K] renormalised scores
  uint32_t* words_out;         // logits path: [T, K] resolved route words for the down kernel
  uint32_t* status;
  uint64_t* trace;             // optional phase timestamps, 8 per block
  uint32_t tokens, slots, hidden, inter, experts, has_shared;
  int act_dtype;
  float blend;
};

// The hyper-connection injection of a branch output y [T, H] into hc residual
// streams (compile_glue.py:32-35): out[t, j*H + h] = round(hidden[t, j*H + h]
// + round(y[t, h] * weights[t, j])), activation dtype.  out == nullptr: off.
constexpr uint32_t kMaxStreams = 8;
struct Inject {
  const void* hidden;          // [T, hc * H]
  const void* weights;         // [T, hc]
  void* out;                   // [T, hc * H], may be `hidden`
  uint32_t hc;
};

struct DownLaunch {
  const void* act;             // [T, S, I]
  const uint32_t* routes;      // [T, K]
  const int32_t* slot_table;
  ProjPtrs down;
  ProjPtrs shared_down;        // internal shared expert (slot K) when has_shared
  const void* shared_sig;      // [T] sigmoid(shared gate), activation dtype
  PoolDev pool;
  PoolDev stream;
  const void* scores;          // [T, K] or null -> per-slot outputs
  int score_dtype;
  const void* shared_y;        // [T, H]
  const void* shared;          // [T, H]
  const void* shared_gate;     // [T]
  void* out;
  uint32_t* status;
  uint64_t* trace;             // optional phase timestamps, 8 per block
  uint32_t tokens, slots, hidden, inter, experts, has_shared;
  int act_dtype;
  // Last, so that the fields above keep the kernel-argument offsets the
  // kernel's scalar loads are scheduled around.
  Inject inject;               // optional injection of the combined rows into residual streams
  uint32_t generic;            // 1: generic combine (products rounded before the slot sum)
};

// ---------------------------------------------------- fused decode (T = 1) --
// The one-token pipelines are built only on request (A/B measurement).
#ifndef VM_FUSED_PIPELINES
#define VM_FUSED_PIPELINES 0
#endif
// A decode call of one token (fused.hip): the front (router logits, the
// shared expert's gate/up + SwiGLU and its sigmoid gate) and one grid of a
// block per CU for the routed experts: either gate/up only, followed by the
// down kernel, or gate/up and every slot's down rows with the activations
// handed over through tagged words (two launches).
constexpr int kFusedMaxGateUp = 4;     // gate/up items per wave of the experts grid
constexpr int kFusedMaxDown = 4;       // down items per wave
constexpr uint32_t kFusedMaxSlots = 11;    // top_k (<= 10) + the shared expert
constexpr uint32_t kFusedMaxInter = 2048;
// Hand-off word w lives at tag_index(w): every 128-byte line of 32 words on a
// 4 KiB page of its own, so the reads of every block spread over the memory
// channels instead of queueing on the few that one dense array maps to.
constexpr uint32_t kTagLineWords = 32;
constexpr uint32_t kTagLineStride = 1024;
__host__ __device__ inline size_t tag_index(uint32_t w) {
  return static_cast<size_t>(w / kTagLineWords) * kTagLineStride + (w % kTagLineWords);
}
__host__ __device__ inline size_t tag_words(uint32_t count) {
  return static_cast<size_t>((count + kTagLineWords - 1) / kTagLineWords) * kTagLineStride;
}

struct FusedLaunch {
  const uint16_t* x;           // [H] bf16
  const uint16_t* router;      // [E, H] bf16
  const float* router_bias;    // optional [E]
  float* logits;               // [E], rounded to bf16
  ProjPtrs sh_gate, sh_up, sh_down, sh_seg;  // shared expert and its H -> 1 gate (has_shared)
  uint16_t* sh_act;            // [I] SwiGLU of the shared expert
  uint16_t* sh_sig;            // [1] sigmoid of the shared gate
  const int32_t* routes;       // [K] expert ids chosen elsewhere (device LRU); null: select from logits
  const uint16_t* route_scores;  // [K] their bf16 scores
  const int32_t* slot_table;   // expert -> pool slot, or null for dense banks
  PoolDev pool;
  ProjPtrs gate, up, down;     // dense routed banks
  uint32_t* act_tag;           // two launches: [K, I] hand-off words (1 << 16 | bf16), zeroed by the front
  uint16_t* act;               // three launches: [K + 1, I] activations (the shared expert's at K)
  uint32_t* words_out;         // three launches: [K] route words for the down kernel
  uint16_t* out;               // [H]
  int32_t* inds_out;           // optional [K]
  uint16_t* scores_out;        // optional [K]
  uint32_t* status;            // bit 0: unresolved expert, bit 5: hand-off wait gave up
  uint64_t* trace;
  Inject inject;
  uint32_t hidden, inter, experts, slots, has_shared, generic;
  float blend;
  uint32_t gu_items, dn_tiles;  // gate/up row groups and down row tiles of the experts grid
};

// Launch shape of the fused decode for a layer shape, or false when the
// three-launch path must run it (grid = blocks of the experts kernel).
bool fused_plan(uint32_t hidden, uint32_t inter, uint32_t slots, uint32_t has_shared, uint32_t experts,
                uint32_t blocks, FusedLaunch& p);
hipError_t launch_fused_front(const FusedLaunch& p, hipStream_t stream);
// down: the two-launch experts grid; otherwise its gate/up part only
hipError_t launch_fused_experts(const FusedLaunch& p, uint32_t blocks, bool down, hipStream_t stream);

// ------------------------------------------------------ device-side LRU --
constexpr uint32_t kLruMaxRouted = 80;  // VM_LAYER_MAX_TOKENS * MAX_TOP_K
constexpr int kLruThreads = 1024;       // one block runs the selection and the assign
constexpr int kLruSlotsPerThread = 32;  // queue entries each thread holds in registers
constexpr uint32_t kLruMaxSlots = kLruThreads * kLruSlotsPerThread;
constexpr uint32_t kNoRecord = 0xffffffffu;

// assign() of one decode call on the device state (one block).
struct LruLaunch {
  int32_t* slot_table;         // [layers, experts]
  int32_t* slot_owner;         // [slots]
  int32_t* lru_order;          // [order_len] slot ids, least recently used first
  uint64_t* counters;          // [4 + 4 * layers]
  const int32_t* host_row;     // [layers, experts]
  uint32_t* fill_count;        // [1] misses of the call
  uint32_t* fill_src;          // [routed] host row of miss m (kNoRecord: none)
  uint32_t* fill_dst;          // [routed] slot of miss m
  uint32_t* status;
  uint64_t host_records;
  uint32_t routed, experts, layers, layer, slots, order_len;
};

// Copy of the missed records from pinned host memory into their slots.
struct FillLaunch {
  const uint32_t* count;
  const uint32_t* src;
  const uint32_t* dst;
  const uint8_t* host;         // device-accessible address of the pinned store
  uint64_t host_stride, host_records;
  uint8_t* pool;
  uint64_t header, stride, pool_records, record_bytes;
};

// Softmax/top-k of up to kLruWaves tokens and the LRU assign of their routed
// ids, one block (decode.hip).
hipError_t launch_select_lru(const SelectLaunch& p, const LruLaunch& l, hipStream_t stream);
hipError_t launch_fill(const FillLaunch& p, hipStream_t stream);

// ---------------------------------------------------------- grouped path --
#ifndef VM_GROUPED_ROWS
#define VM_GROUPED_ROWS 64
#endif
#ifndef VM_GROUPED_ROWS_DN
#define VM_GROUPED_ROWS_DN 48
#endif
// rows per grouped GEMM tile (16, 32, 48 or 64): gate/up (and the router
// GEMM), and the down projection, whose short K (the intermediate size) runs
// best with more, shorter tiles at two blocks per CU
#ifndef VM_GROUPED_ROWS_RT
#define VM_GROUPED_ROWS_RT 64
#endif
constexpr int kGroupedRows = VM_GROUPED_ROWS;
// Tall gate/up and down tiles: for calls whose routed experts average more
// rows than one tile of the usual height holds (64 gate/up, 48 down: from
// about 3072 rows at 512 experts top-10), so that a group takes fewer tiles
// and its weights are dequantised that much less often; the blocks then run
// two per CU instead of three (gate/up) and one instead of two (down).  The
// shared expert's down takes them above 48 rows of its own.
#ifndef VM_GROUPED_ROWS_TALL
#define VM_GROUPED_ROWS_TALL 96
#endif
constexpr int kGroupedRowsTall = VM_GROUPED_ROWS_TALL;
constexpr int kGroupedRowsDown = VM_GROUPED_ROWS_DN;
constexpr int kGroupedRowsRouter = VM_GROUPED_ROWS_RT;  // router GEMM tiles (no sort: rows in order)
constexpr uint32_t kNoRow = 0xffffffffu;  // pair without a row (invalid expert id)
enum : int { kEpiSwiglu = 0, kEpiRows = 1, kEpiLogits = 2 };

// Grouped GEMM over row tiles of expert groups: out[row, n] from A rows x
// dequantised weights (or bf16 router weights).
struct GroupedLaunch {
  const uint16_t* a;           // bf16 activations, a_stride elements per row
  const uint32_t* row_token;   // A row of sorted row r is row_token[r] (null: r)
  const uint32_t* row_off;     // [groups + 1] first sorted row of every group
  const uint2* tiles;          // (group, first row in group); null: one group of `rows` rows
  const uint32_t* tile_count;
  uint32_t rows;
  const int32_t* slot_table;   // expert -> pool slot, or null
  PoolDev pool;
  PoolDev stream;
  ProjPtrs dense[2];           // routed banks [E, N, K/8], projection 0 and 1
  ProjPtrs shared[2];          // group == experts: the shared expert
  int part[2];                 // record part of each projection (0 gate, 1 up, 2 down)
  const uint16_t* bf16_weight; // router [N, K]
  const float* bias;           // router, optional [N]
  void* out;
  uint32_t* status;
  uint64_t* trace;             // phase trace of the 16-row tile kernels (diagnostics), or null
  uint32_t k_dim, n_dim, experts, a_stride;
  uint32_t a_rows;             // rows of the A matrix: the chunked GEMM addresses it with 32-bit byte offsets
  uint32_t spb;                // column slices per block (set by launch_grouped)
  uint32_t tile_rows;          // rows per tile of `tiles`: 0 the instance's own, or kGroupedRowsTall (gate/up)
  bool weights_once;           // most groups hold one row tile: stream the weights past the L2
  // router GEMM only: block 0 zeroes zero_count words at zero_words (the
  // counters of the sort that follows the select)
  uint32_t* zero_words;
  uint32_t zero_count;
};

// Router logits of grouped calls as a bf16 GEMM streamed through an LDS ring
// (router_gemm.hip): fp32 [rows, n_dim] = round_bf16(a . bf16_weight^T +
// bias), block 0 zeroing zero_words.  Shapes: k_dim 1024, 2048 or 4096,
// n_dim a multiple of 64, a_stride == k_dim.
bool router_gemm_supported(uint32_t k_dim, uint32_t n_dim);
hipError_t launch_router_gemm(const GroupedLaunch& p, hipStream_t stream);

struct SortLaunch {
  const int32_t* inds;         // [tokens, slots]
  uint32_t* row_off;           // [groups + 1]
  uint2* tiles;                // tile_rows-row tiles (gate/up)
  uint32_t* tile_count;
  uint2* tiles_dn;             // tile_rows_dn-row tiles (down)
  uint32_t* tile_count_dn;
  uint32_t* counts;            // [1024] scratch of the multi-block sort: rows per group
  uint32_t* cursors;           // [1024] scratch of the multi-block sort: next free row per group
  uint32_t* row_token;         // [rows]
  uint32_t* pair_row;          // [tokens * slots]
  uint32_t* status;
  uint32_t tokens, slots, experts, shared_rows;
  uint32_t tile_rows, tile_rows_dn;  // rows per tile of the two lists
};

struct CombineLaunch {
  const uint16_t* rows;        // expert output rows [rows, hidden] bf16
  const uint32_t* pair_row;    // [tokens * slots]
  const void* scores;          // [tokens, slots]
  int score_dtype;
  const uint32_t* shared_first; // row of token 0's shared expert output in `rows` (with shared_sig)
  const uint16_t* shared_rows; // or the shared expert's output rows [tokens, hidden] bf16 (with shared_sig)
  const void* shared_sig;      // [tokens] bf16
  const void* shared_y;        // or a finished shared term [tokens, hidden] bf16
  void* out;                   // [tokens, hidden] bf16
  uint32_t tokens, slots, hidden;
  int mode;                    // 0 fused combine, 1 generic combine, 2 per-slot rows
  Inject inject;               // modes 0 and 1: optional injection into residual streams
};

// Upper bound of the tiles of `tile_rows` rows over `groups` groups holding `rows` rows.
uint32_t grouped_max_tiles(uint32_t rows, uint32_t groups, uint32_t tile_rows);
hipError_t launch_grouped(int epi, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream);
// The 16-row tile kernels of small calls (see k_rows); false when K is above
// their LDS bound.
constexpr int kRowsTile = 16;
bool rows_supported(uint32_t k_dim);
hipError_t launch_rows(int epi, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream);
// Calls up to this many (token, slot) pairs sort in one block.
constexpr uint32_t kSortOneBlockPairs = 4096;
hipError_t launch_sort(const SortLaunch& p, hipStream_t stream);
// The sort when p.counts and p.cursors were zeroed before it (by the router
// GEMM): per-block histograms into the counts, then one launch lays out the
// rows and tiles and scatters the pairs.
hipError_t launch_sort_counted(const SortLaunch& p, hipStream_t stream);
hipError_t launch_grouped_combine(const CombineLaunch& p, hipStream_t stream);
hipError_t launch_shared_gate(const uint16_t* x, const ProjPtrs& seg, uint16_t* sig, uint32_t tokens,
                              uint32_t hidden, hipStream_t stream);

hipError_t launch_front(const FrontLaunch& p, hipStream_t stream);
hipError_t launch_select(const SelectLaunch& p, hipStream_t stream);
hipError_t launch_gateup(const GateUpLaunch& p, hipStream_t stream);
hipError_t launch_down(const DownLaunch& p, hipStream_t stream);
hipError_t launch_weighted_combine(const void* values, const void* scores, void* out, uint32_t tokens,
                                   uint32_t slots, uint32_t hidden, int act_dtype, int score_dtype,
                                   hipStream_t stream);

// Shape support of the decode kernels.
bool gateup_supported(uint32_t hidden);
bool down_supported(uint32_t inter, uint32_t slots_total, int act_dtype);

// Kernel timing (api.hip): when timing is on, returns the start/stop events
// to attach to the next launch of `family` (hipExtLaunchKernelGGL stamps them
// when the kernel starts and ends) and queues them for vm_timing_read.
bool timing_events(const char* family, hipEvent_t* start, hipEvent_t* stop);
// Phase-trace records for a launch of `blocks` blocks (null when tracing is off or full).
uint64_t* trace_reserve(uint32_t blocks);

// Phase timestamps: thread 0 of a block keeps them and writes one record of
// 16 uint64: [kernel id, block, t0 .. t11, 0, 0].
constexpr int kTraceWords = 16;
constexpr int kTraceMarks = 12;
struct PhaseTrace {
  uint64_t t[kTraceMarks] = {};
  __device__ __forceinline__ void mark(int i) { t[i] = __builtin_amdgcn_s_memrealtime(); }
  __device__ __forceinline__ void write(uint64_t* trace, uint32_t kernel_id, uint32_t block) const {
    uint64_t* r = trace + static_cast<size_t>(block) * kTraceWords;
    r[0] = kernel_id;
    r[1] = block;
    for (int i = 0; i < kTraceMarks; ++i) r[2 + i] = t[i];
    r[14] = r[15] = 0;
  }
};

// ---------------------------------------------------------- decoder glue --
constexpr uint32_t kHcMaxRow = 16384;     // hc * hidden
constexpr uint32_t kHcMaxLowrank = 256;

// The hyper-connection before a branch (glue.hip).
struct HcLaunch {
  const void* hidden;          // [T, n] the residual streams, n = hc * hidden
  const void* norm_weight;     // [n] hc_norm gain
  ProjPtrs down, up, inj;      // [lowrank, n/8], [n, lowrank/8], [hc, n/8] Q4/G32
  void* normed;                // [T, n]
  void* d;                     // [T, lowrank]
  void* mixed;                 // [T, hidden]
  void* weights;               // [T, hc]
  float eps;
  uint32_t tokens, width, hc, n, lowrank, norm_group, one_centered;  // width = hidden size
  int act_dtype;
};

hipError_t launch_hyper_mix(const HcLaunch& p, hipStream_t stream);

}  // namespace vm
