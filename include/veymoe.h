/*
 * veymoe.h - C ABI of the MI355X (gfx950) routed-expert MoE layer.
 *
 * One SwiGLU mixture-of-experts layer with 4-bit affine, group-32 quantized
 * experts in the MLX packed layout:
 *   weight  uint32 [E, out, in/8]    nibble k of a row sits at bits 4*(k&7) of word k>>3
 *   scales  bf16   [E, out, in/32]   (passed as uint16 bit patterns)
 *   biases  bf16   [E, out, in/32]
 *   dequantized w = scale * q + bias
 *
 * Every pointer is a DEVICE pointer unless the field says "host".  The caller
 * owns all memory; the library never allocates or frees caller memory.  Calls
 * are asynchronous on the given HIP stream.  Return value: 0 on success or a
 * negative VM_E* code; the message of the last failure on the calling thread
 * is available from vm_last_error().
 *
 * Reference interfaces (joyboyreturns/Veystrix-Core) these entry points replace:
 *   vm_moe_execute     MetalMoEExecutor.execute         models/flashnext/metal_runtime.py:799-974
 *                      flashnext_native_moe_execute     models/flashnext/tests/bench/metal_runtime_native.mm:258-395
 *   vm_router_topk     router softmax/top-k/renorm      models/flashnext/adaptive_topk.py:59-65,257-262
 *                                                       models/flashnext/compiled.py:61-71
 *   vm_moe_layer       _moe_call                        models/flashnext/adaptive_topk.py:54-293
 *                      (rows <= 8: custom-kernel branch :289-293; rows > 8: generic branch :275-278)
 *   vm_moe_grouped     _one_pass/_issue gather_qmm path models/flashnext/expert_cache.py:1949-2037 (rows > 8)
 *   vm_weighted_combine weighted_combine                models/flashnext/metal_runtime.py:145-191
 *   vm_pool_stage      ExpertPool.fill/_fill_part       models/flashnext/expert_pool.py:201-220,258-287
 *   vm_moe_layer_lru   _pool_pass (route sync, assign, fill, execute)
 *                                                       models/flashnext/expert_cache.py:1709-1772,1842-1947
 *                                                       models/flashnext/expert_pool.py:123-159,201-220
 *   vm_hyper_mix       the branch's hyper-connection    models/flashnext/qwen4_verifier.py:20-33
 *                      (hc_norm RMSNorm)                models/flashnext/patch_rmsnorm.py:108-135
 *   VmLayerArgs.inject_*  _inject after the branch      models/flashnext/compile_glue.py:32-41
 *   vm_available       flashnext_native_available       metal_runtime_native.mm:196-201
 *   vm_last_error      flashnext_native_get_last_error  metal_runtime_native.mm:203-209
 */
#ifndef VEYMOE_H
#define VEYMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VM_ABI_VERSION 3

/* status codes (0 = ok) */
#define VM_OK 0
#define VM_EINVAL -1      /* malformed argument or shape contract violation */
#define VM_EUNSUPPORTED -2 /* valid but not implemented for this shape */
#define VM_EHIP -3        /* a HIP runtime call failed */
#define VM_EWORKSPACE -4  /* workspace too small */

/* element types of activations, scores and outputs */
#define VM_BF16 0
#define VM_F32 1

/* route words (uint32): bit 31 set -> record `word & 0x7fffffff` of the pool
 * view; clear -> expert index into the dense projection arrays.  When a slot
 * table is given, route words are expert ids and the table maps each to a pool
 * slot (-1 = not resident).  Same encoding as the reference's SLOT_BIT
 * (models/flashnext/expert_pool.py:44, metal_runtime.py:198-228). */
#define VM_SLOT_BIT 0x80000000u

/* record parts, in the order of the reference's expert-major record
 * (models/flashnext/slab_pack.py:96-149, expert_pool.py:45-49) */
enum {
  VM_PART_GATE_W = 0, VM_PART_GATE_S, VM_PART_GATE_B,
  VM_PART_UP_W, VM_PART_UP_S, VM_PART_UP_B,
  VM_PART_DOWN_W, VM_PART_DOWN_S, VM_PART_DOWN_B,
  VM_PARTS
};

/* One quantized projection stored as dense expert-major arrays.  All three
 * pointers may be NULL when every route addresses the pool. */
typedef struct VmQ4Proj {
  const uint32_t* weight; /* [E, out, in/8] */
  const uint16_t* scales; /* [E, out, in/group] bf16 bits */
  const uint16_t* biases; /* [E, out, in/group] bf16 bits */
} VmQ4Proj;

/* A byte region of fixed-stride expert records (the expert pool, or a slab
 * pack: models/flashnext/expert_pool.py:78-117).  Record r starts at
 * base + header_size + r * record_stride (64-bit offsets). */
typedef struct VmPoolView {
  const uint8_t* base;
  uint64_t header_size;
  uint64_t record_stride;
  uint64_t part_offset[VM_PARTS];
  uint32_t records; /* records addressable through this view */
  uint32_t reserved;
} VmPoolView;

/* vm_moe_execute: gate projection, up projection + SwiGLU, down projection and,
 * when `scores` is given, the router-score combine plus an optional shared
 * term.  Mirrors MetalMoEExecutor.execute(x, routes, projections, scores=,
 * slab_pack=, shared_y=, shared=, shared_gate=, pool_activation=, return_all=).
 *
 *   x            [tokens, hidden]              act_dtype
 *   routes       [tokens, slots] uint32 route words
 *   slot_table   optional [expert_count] int32 (see VM_SLOT_BIT)
 *   scores       optional [tokens, slots]      score_dtype
 *   shared_y     optional [tokens, hidden]     act_dtype  (added after the combine)
 *   shared       optional [tokens, hidden]     act_dtype  } added as shared*shared_gate,
 *   shared_gate  optional [tokens]             act_dtype  } rounded to act_dtype
 *   activation_in  optional [tokens, slots, inter] act_dtype: precomputed SwiGLU
 *                  activations (the reference's pool_activation); skips gate/up
 *   activation_out optional [tokens, slots, inter]: receives the activations
 *   gate_out/up_out optional [tokens, slots, inter]: raw projections (return_all)
 *   output       [tokens, hidden] when scores != NULL, else [tokens, slots, hidden];
 *                may be NULL when activation_out is given: gate/up/SwiGLU only
 *                (the reference's pool_activations, metal_runtime.py:783-797)
 *   status       optional device uint32: OR-ed with 1 when a route or slot is
 *                out of range (that slot then contributes zeros)
 *   workspace    device scratch of at least vm_moe_execute_workspace() bytes
 */
typedef struct VmMoeArgs {
  const void* x;
  VmQ4Proj gate, up, down;
  VmPoolView pool;
  VmPoolView stream; /* optional: routes without VM_SLOT_BIT address record
                        `word` here instead of the dense arrays (the reference's
                        stream pack, metal_runtime.py:202-208); header_size is
                        normally 0 */
  const uint32_t* routes;
  const int32_t* slot_table;
  const void* scores;
  const void* shared_y;
  const void* shared;
  const void* shared_gate;
  const void* activation_in;
  void* activation_out;
  void* gate_out;
  void* up_out;
  void* output;
  uint32_t* status;
  void* workspace;
  uint64_t workspace_bytes;
  uint32_t tokens, slots, hidden_size, inter_size, expert_count, group_size;
  uint32_t act_dtype, score_dtype;
} VmMoeArgs;

/* vm_router_topk: logits = x . router_weight^T (+ optional fp32 logit bias),
 * rounded to act_dtype; gates = softmax in fp32, rounded to act_dtype; the
 * top_k gates by (value descending, expert index ascending); scores = gates of
 * the selection divided by their sum, each step rounded to act_dtype.
 *   inds   [tokens, top_k] int32 out, in selection order
 *   scores [tokens, top_k] act_dtype out (renormalised)
 *   gates  optional [tokens, expert_count] act_dtype out (full softmax) */
typedef struct VmRouterArgs {
  const void* x;
  const uint16_t* weight; /* [expert_count, hidden] bf16 bits */
  const float* logit_bias; /* optional [expert_count] */
  int32_t* inds;
  void* scores;
  void* gates;
  void* workspace;
  uint64_t workspace_bytes;
  uint32_t tokens, hidden_size, expert_count, top_k;
  uint32_t act_dtype;
  float renorm_blend; /* the reference's FLASHNEXT_RENORM_BLEND; 1 = plain renorm */
} VmRouterArgs;

/* vm_moe_layer: one whole MoE layer: router top-k, device-side expert -> pool
 * slot resolution through slot_table, the shared expert (gate/up/SwiGLU/down)
 * and its sigmoid gate, the routed experts, and the combine.
 * tokens <= VM_LAYER_MAX_TOKENS (the reference's custom-kernel bound,
 * metal_runtime.py:26): decode kernels and the fused combine
 *   y = round(round(sum_j round(down_j) * score_j) + round(sigmoid(g_s) * shared)).
 * More tokens (bf16): the grouped path (router GEMM, device token-by-expert
 * sort, MFMA grouped gate/up and down) and the generic combine of
 * adaptive_topk.py:275-278
 *   y = round(round(sum_j round(round(down_j) * score_j)) + round(sigmoid(g_s) * shared)).
 * More tokens in fp32: the decode kernels over chunks of VM_LAYER_MAX_TOKENS.
 * Routed experts come from the pool view (slot_table) or, when slot_table is
 * NULL, from the dense arrays in `gate/up/down` indexed by expert id.
 * shared_inter == 0 means no shared expert. */
#define VM_LAYER_MAX_TOKENS 8
typedef struct VmLayerArgs {
  const void* x;                 /* [tokens, hidden] */
  void* output;                  /* [tokens, hidden] */
  const uint16_t* router_weight; /* [expert_count, hidden] bf16 */
  const float* router_bias;      /* optional [expert_count] */
  VmQ4Proj gate, up, down;       /* dense routed experts (used when slot_table == NULL) */
  VmPoolView pool;
  const int32_t* slot_table;     /* [expert_count] or NULL */
  VmQ4Proj shared_gate_proj, shared_up_proj, shared_down_proj; /* [1, ...] */
  VmQ4Proj shared_expert_gate;   /* [1, 1, hidden/8]: the H -> 1 quantized gate */
  int32_t* inds_out;             /* optional [tokens, top_k] */
  void* scores_out;              /* optional [tokens, top_k] act_dtype */
  uint32_t* status;              /* optional, see VmMoeArgs */
  void* workspace;
  uint64_t workspace_bytes;
  uint32_t tokens, hidden_size, inter_size, shared_inter, expert_count, top_k, group_size;
  uint32_t act_dtype;
  float renorm_blend;
  uint32_t phases; /* VM_PHASE_* bits; 0 means both.  A router-only call leaves
                      inds/scores (inds_out/scores_out or the workspace) for a
                      later experts-only call with the same workspace, so the
                      host can resolve pool misses in between. */
  /* Optional hyper-connection injection of the layer output y into the
   * residual streams, in the experts' final epilogue (replaces the decoder's
   * _inject, compile_glue.py:32-35):
   *   inject_out[t, j*H + h] = round(inject_hidden[t, j*H + h]
   *                                  + round(y[t, h] * inject_weights[t, j]))
   * for j < hc_count (1..VM_MAX_STREAMS), activation dtype; `output` still
   * receives y.  inject_out may equal inject_hidden.  NULL inject_out: off. */
  const void* inject_hidden;     /* [tokens, hc_count * hidden] */
  const void* inject_weights;    /* [tokens, hc_count] */
  void* inject_out;              /* [tokens, hc_count * hidden] */
  uint32_t hc_count;
  /* Decode calls (tokens <= VM_LAYER_MAX_TOKENS): VM_COMBINE_FUSED, or
   * VM_COMBINE_GENERIC for the generic combine formula above.  The reference
   * takes the generic one for layer 0 (metal_combines_scores is False there,
   * expert_cache.py:1434-1443; adaptive_topk.py:271-278).  Grouped calls
   * always combine generically. */
  uint32_t combine;
  /* Optional [tokens, expert_count] activation dtype: the softmax gates of
   * every expert, written by router-only calls (phases == VM_PHASE_ROUTER).
   * The host's adaptive top-k (adaptive_topk.py:76-235) reads the selected
   * experts' gates from here before it rewrites the routes for the experts
   * call.  No counterpart in the reference's C surface: MLX hands the host
   * the gates array itself. */
  void* gates_out;
} VmLayerArgs;
#define VM_COMBINE_FUSED 0u
#define VM_COMBINE_GENERIC 1u
#define VM_PHASE_ROUTER 1u
#define VM_PHASE_EXPERTS 2u
#define VM_MAX_STREAMS 8

/* vm_hyper_mix: the hyper-connection in front of a decoder branch, for any
 * token count (qwen4_verifier.py:20-33, Qwen4ExpGatedResidual; the norm is
 * patch_rmsnorm.py:108-135).  With n = hc_count * hidden_size:
 *   normed  = rms_norm(hidden)            fp32 mean of squares over the whole
 *             row (norm_group 0) or groups of norm_group; gain = weight
 *             (one_centered) or 1 + weight
 *   d       = silu(mix_down . normed / hc_count)          [lowrank]
 *   mixed   = mean_j(sigmoid(mix_up . d)_j * normed_j)    [hidden], the branch input
 *   weights = 2 * sigmoid(inject . normed / hc_count)     [hc_count]
 * Q4/G32 projections in the vector form, every step rounded to the
 * activation dtype.  Requirements: n % 64 == 0, n <= 16384, norm_group 0 or
 * a multiple of 64 dividing n, lowrank a multiple of 32 up to 256,
 * hc_count 1..VM_MAX_STREAMS, 16-byte aligned hidden rows.  The workspace
 * (vm_hyper_mix_workspace bytes) receives normed and d unless `normed` is
 * given. */
typedef struct VmHyperArgs {
  const void* hidden;            /* [tokens, n] the residual streams */
  const void* norm_weight;       /* [n] hc_norm gain, activation dtype */
  VmQ4Proj mix_down;             /* [lowrank, n/8] */
  VmQ4Proj mix_up;               /* [n, lowrank/8] */
  VmQ4Proj inject;               /* [hc_count, n/8] */
  void* mixed;                   /* out [tokens, hidden] */
  void* weights;                 /* out [tokens, hc_count] */
  void* normed;                  /* optional out [tokens, n] */
  void* workspace;
  uint64_t workspace_bytes;
  uint32_t tokens, hidden_size, hc_count, lowrank, norm_group, one_centered;
  uint32_t act_dtype;
  float eps;
} VmHyperArgs;

/* vm_moe_layer_lru: the decode layer (tokens <= VM_LAYER_MAX_TOKENS) over an
 * expert pool whose LRU state lives on the device, so the call never waits for
 * the host.  It replaces the reference's per-layer route sync + host
 * ExpertPool.assign + fill (expert_cache.py:1738-1749, 1842-1947;
 * expert_pool.py:123-159, 201-220): the router selects on the device, one
 * block applies assign() to the routed ids of the call, missed records are
 * copied by a kernel straight from pinned host memory into their new slots,
 * then the experts run through the updated slot table.
 *
 * assign() semantics, exactly as the reference's LRU: the distinct experts of
 * the call in first-seen order (tokens in order, slots in rank order); hits
 * move to the most recent end in that order; then each miss, in that order,
 * takes the next victim: free slots first (in the order the reference's free
 * list pops them), then the least recently used key, whose table entry is
 * cleared.  Recency is one queue of slot ids, lru_order: the free slots in
 * pop order, then the resident slots from least to most recently used (the
 * reference's free list followed by its OrderedDict).  A call's victims are
 * the first misses-many entries of the queue that are not hits; the queue
 * then holds the remaining non-hit entries, the hits in first-seen order and
 * the victims in miss order.
 *
 * State (device memory owned by the caller, updated in place):
 *   slot_table  [layers, expert_count] int32: expert -> slot, -1 = absent
 *               (row `layer` replaces VmLayerArgs.slot_table, which is ignored)
 *   slot_owner  [slots] int32: layer * expert_count + expert, -1 = free
 *   lru_order   [order_len] int32: every candidate slot once (slots outside
 *               the queue are never handed out)
 *   counters    [4 + 4 * layers] uint64: distinct ids assigned (hits plus
 *               misses), distinct hits, distinct misses, routed hits (routed
 *               positions minus distinct misses, the reference's
 *               StreamingSwitchGLU.hits); then per layer: distinct hits,
 *               distinct misses, routed hits, routed ids
 *   host_row    [layers, expert_count] int32: row of the expert's record in
 *               host_store (-1: no record)
 *   host_store  pinned host memory (hipHostMalloc), host_records rows of
 *               host_stride bytes; rows are read by the GPU over the host link
 * slots must equal VmLayerArgs.pool.records, order_len must be at most slots
 * and at least tokens * top_k.  A miss whose expert has no host record is left
 * unfilled and sets status bit 4; a routed id outside 0..expert_count-1 is
 * skipped and sets status bit 8.  Status bit 16: a queue with an entry outside
 * 0..slots-1 or without every hit slot exactly once leaves the state unchanged
 * (nothing mapped, nothing filled); a queue with fewer non-hit entries than
 * misses maps only the misses it can.  Calls that overlap on one state race:
 * issue them on one stream. */
typedef struct VmDeviceLru {
  int32_t* slot_table;
  int32_t* slot_owner;
  int32_t* lru_order;
  uint64_t* counters;
  const int32_t* host_row;
  const void* host_store;
  uint64_t host_stride;
  uint64_t host_records;
  uint32_t layers;
  uint32_t layer;
  uint32_t slots;
  uint32_t order_len;
} VmDeviceLru;

/* vm_moe_grouped: the expert block of the grouped path for any token count
 * with given routes (SwitchGLU over expert ids, expert_cache.py:1949-2037):
 * token-by-expert sort on the device, MFMA grouped gate/up/SwiGLU and down
 * over every expert's rows, then the combine (bf16 activations).
 * combine_mode 0: fused form (fp32 sum of round(down)*score, as vm_moe_layer)
 * combine_mode 1: generic form of adaptive_topk.py:275-278,
 *   y = round(round(sum_j round(round(down_j) * score_j)) + shared_y)
 * combine_mode 2: no combine; output [tokens, top_k, hidden] = round(down_j)
 *   (SwitchGLU without scores, the reference's rows > 8 return shape).
 * Routes are expert ids resolved through slot_table, or dense indices.  An id
 * outside 0..expert_count-1 contributes nothing and sets status bit 2. */
typedef struct VmGroupedArgs {
  const void* x;                 /* [tokens, hidden] */
  const int32_t* inds;           /* [tokens, top_k] expert ids */
  const void* scores;            /* [tokens, top_k] act_dtype */
  VmQ4Proj gate, up, down;
  VmPoolView pool;
  const int32_t* slot_table;
  const void* shared_y;          /* optional [tokens, hidden] act_dtype */
  void* output;                  /* [tokens, hidden] */
  uint32_t* status;
  void* workspace;
  uint64_t workspace_bytes;
  uint32_t tokens, top_k, hidden_size, inter_size, expert_count, group_size;
  uint32_t act_dtype, combine_mode;
} VmGroupedArgs;

int vm_abi_version(void);
/* 1 when a gfx950 device is usable by this library, else 0. */
int vm_available(void);
/* Copies the calling thread's last error message (NUL-terminated). */
int vm_last_error(char* buf, size_t len);

uint64_t vm_moe_execute_workspace(uint32_t tokens, uint32_t slots, uint32_t inter_size, uint32_t act_dtype);
int vm_moe_execute(const VmMoeArgs* args, void* stream);

uint64_t vm_router_workspace(uint32_t tokens, uint32_t expert_count);
int vm_router_topk(const VmRouterArgs* args, void* stream);

uint64_t vm_moe_layer_workspace(uint32_t tokens, uint32_t top_k, uint32_t hidden_size, uint32_t inter_size,
                                uint32_t shared_inter, uint32_t expert_count, uint32_t act_dtype);
int vm_moe_layer(const VmLayerArgs* args, void* stream);
/* Workspace: vm_moe_layer_workspace() of the same shape. */
int vm_moe_layer_lru(const VmLayerArgs* args, const VmDeviceLru* lru, void* stream);

/* vm_moe_layer_static: vm_moe_layer with the library's own scratch in place
 * of args->workspace / workspace_bytes (both ignored).  It allocates nothing
 * (no hipMalloc, hipFree or allocating library call), for callers that cannot
 * allocate: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  No counterpart in the reference.  The scratch is a static
 * device array of VM_STATIC_SCRATCH_BYTES on each GPU the library runs on,
 * held until the process ends; a call whose vm_moe_layer_workspace() exceeds
 * it fails with VM_EWORKSPACE.  Every call on one GPU shares that GPU's
 * array and leaves its contents behind: calls that overlap on one GPU (two
 * streams, two threads) race.  A router-only call followed by an
 * experts-only call (VM_PHASE_*) works as with one workspace, provided no
 * other call on that GPU runs in between.  The stream must belong to the
 * current device. */
#define VM_STATIC_SCRATCH_BYTES (4ull << 20)
int vm_moe_layer_static(const VmLayerArgs* args, void* stream);

/* The hyper-connection before a branch (see VmHyperArgs): two launches. */
uint64_t vm_hyper_mix_workspace(uint32_t tokens, uint32_t hc_count, uint32_t hidden_size, uint32_t lowrank,
                                uint32_t act_dtype);
int vm_hyper_mix(const VmHyperArgs* args, void* stream);

uint64_t vm_moe_grouped_workspace(uint32_t tokens, uint32_t top_k, uint32_t hidden_size,
                                  uint32_t inter_size, uint32_t expert_count, uint32_t act_dtype);
int vm_moe_grouped(const VmGroupedArgs* args, void* stream);

/* out[t, h] = sum_j expert_outputs[t, j, h] * scores[t, j] in fp32, written in
 * act_dtype; the normal form of weighted_combine (metal_runtime.py:145-191). */
int vm_weighted_combine(const void* expert_outputs, const void* scores, void* out,
                        uint32_t tokens, uint32_t slots, uint32_t hidden_size,
                        uint32_t act_dtype, uint32_t score_dtype, void* stream);

/* Miss staging: copy `count` whole expert records from pinned host memory
 * (src_host + src_index[i] * src_stride) to pool record dst_slot[i]
 * (pool_base + header_size + dst_slot[i] * record_stride), record_bytes each,
 * with hipMemcpyAsync on `stream`.  src_index and dst_slot are HOST arrays;
 * indices must be below src_records / pool_records.  Runs that are
 * consecutive on both sides are merged into one copy, as the reference merges
 * consecutive rows into one preadv (expert_pool.py:207-212).
 * Replaces the nine per-part preadv rows of ExpertPool.fill
 * (expert_pool.py:258-287) with one DMA per record run. */
int vm_pool_stage(void* pool_base, uint64_t header_size, uint64_t record_stride, uint64_t pool_records,
                  const void* src_host, uint64_t src_stride, uint64_t src_records, uint64_t record_bytes,
                  const int64_t* src_index, const int64_t* dst_slot, uint32_t count,
                  void* stream);

/* vm_decode_pipeline: the kernels of one-token bf16 decode calls (vm_moe_layer
 * and vm_moe_layer_lru), process-wide:
 *   0 (the default): the multi-token kernels (router, gate/up with the
 *     shared expert, down);
 *   1: the one-token front (router logits, the shared expert's gate/up and
 *     its sigmoid gate), a gate/up grid of one block per CU over the routed
 *     experts, and the down + combine kernel;
 *   2: two launches, the front and one experts grid that hands its gate/up
 *     activations to its down rows through tagged words.
 * All three give the same bits.  -1 queries.  Returns the previous setting.
 * Pipelines 1 and 2 were measured slower than 0 and are compiled only into a
 * library built with -DVM_FUSED_PIPELINES=1; otherwise modes 1 and 2 return
 * VM_EUNSUPPORTED.  No counterpart in the reference: it is for A/B
 * measurement and the parity tests of the pipelines. */
int vm_decode_pipeline(int mode);

/* Per-kernel event timing over a window of calls (for rooflines).  While
 * enabled, every kernel the library launches is bracketed by hipEvents on its
 * stream; vm_timing_read returns the summed milliseconds and launch count of
 * the kernel family `name` ("router", "gateup", "down", "experts",
 * "grouped_gateup", "grouped_down", "sort", "combine"). */
int vm_timing_enable(int enabled);
int vm_timing_read(const char* name, double* total_ms, uint64_t* launches);
int vm_timing_reset(void);

/* Phase trace (diagnostics): while a device buffer is set, the decode
 * kernels write 100 MHz timestamps (s_memrealtime) of their phases, one
 * record of 16 uint64 per block: [kernel id, block, t0 .. t11, 0, 0]; the
 * records of one launch are consecutive, in block order.  Pass NULL to stop.
 * vm_trace_records returns the number of records reserved since the set. */
int vm_trace_set(void* device_buffer, uint64_t bytes);
uint64_t vm_trace_records(void);

#ifdef __cplusplus
}
#endif

#endif /* VEYMOE_H */
