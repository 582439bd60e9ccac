// Decode kernels of the routed-expert MoE layer for gfx950 (wave64).
//
// A decode layer is three launches with no cross-block sync inside a kernel
// (a device-scope release writes back the XCD's L2 and costs more than a
// kernel boundary on this part):
//
//   k_front   router logits x . Wr^T (one row per wave, bf16 dot2) and the
//             shared expert's H -> 1 Q4 gate with its sigmoid.
//   k_gateup  in every block of a routed pair, one chooser wave recomputes
//             the token's softmax from the logits, extracts the key of its
//             slot's rank from the lanes' sorted keys by wave maxima
//             (vm_select.h), maps the expert to its slot through the slot
//             table entries it loaded beside the logits, and hands the route
//             word to the block's other wave through LDS.  Every lane then
//             streams gate and up Q4/G32 rows against its activation groups
//             held in registers; SwiGLU runs on the lanes that hold the row
//             sums.  Shared-expert pairs skip the selection.  One block per
//             token publishes the ordered selection (indices, scores, route
//             words) for k_down.
//   k_down    down Q4/G32 GEMV of every slot of a token for a tile of output
//             rows (one slot per wave), then the router-score
//             combine with the shared term after one barrier.
//   k_select  softmax + top-k alone (router entry point, split layer path).
//
// Bandwidth layout: one 16-byte load per lane covers one 32-input group of a
// row (4 packed words); the scale and bias loads of 64 lanes coalesce into one
// 128-byte line per row; activations are read by each lane for its own groups,
// re-paired for v_dot2 with the group sums alongside; row sums use DPP.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "vm_internal.h"
#include "vm_lru.h"
#include "vm_select.h"

namespace vm {

namespace {

constexpr int kBlock = 256;
// router front: waves per block (one router row per wave)
#ifndef VM_FRONT_WAVES
#define VM_FRONT_WAVES 4
#endif
constexpr int kFrontW = VM_FRONT_WAVES;
// block shapes of the full-width (hidden >= 2048) decode GEMVs: output rows per
// lane group in gate/up, row groups per block in down
#ifndef VM_GATEUP_ROWS
#define VM_GATEUP_ROWS 2
#endif
#ifndef VM_DOWN_QUADS
#define VM_DOWN_QUADS 2
#endif
constexpr int kGateupRowsPerLane = VM_GATEUP_ROWS;
#ifndef VM_GATEUP_WAVES
#define VM_GATEUP_WAVES 2
#endif
constexpr int kGuWaves = VM_GATEUP_WAVES;  // waves per gate/up block
constexpr int kGuBlock = kGuWaves * 64;
template <class A, bool GATE = false>
__device__ void select_body(const SelectLaunch& p) {
  __shared__ typename Cand<A>::T s_cand[kMaxCand];
  const uint32_t t = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  GateKeys<A> g;
  float lg[kMaxExpertsPerLane];
  load_logits(p.logits + static_cast<size_t>(t) * p.experts, p.experts, lane, lg);
  if constexpr (GATE) {  // its loads go out with the logits'
    static_assert(std::is_same_v<A, ActBF16>, "the shared gate of bf16 grouped calls");
    const float logit = shared_gate_logit_bf16(p.gate_x + static_cast<size_t>(t) * p.hidden, p.seg, p.hidden, lane);
    if (lane == 0) ActBF16::store(p.shared_sig, t, sigmoid_act<ActBF16>(logit));
  }
  softmax_keys<A>(lg, p.experts, lane, g);
  if (p.gates != nullptr) {
    void* gates = static_cast<char*>(p.gates) + static_cast<size_t>(t) * p.experts * A::kBytes;
#pragma unroll
    for (int m = 0; m < kMaxExpertsPerLane; ++m) {
      const uint32_t e = lane + 64 * m;
      if (e < p.experts) A::store(gates, e, GateKeys<A>::gate(g.k[m]));
    }
  }
  uint32_t e;
  float score;
  rank_selection<A>(g, p.top_k, p.blend, lane, s_cand, e, score);
  if (lane < p.top_k) {
    p.inds[static_cast<size_t>(t) * p.top_k + lane] = static_cast<int32_t>(e);
    A::store(p.scores, static_cast<size_t>(t) * p.top_k + lane, score);
  }
}

__global__ __launch_bounds__(64) void k_select_bf16(SelectLaunch p) { select_body<ActBF16>(p); }
// with the shared expert's sigmoid gate of each token (an instance of its own:
// the gate's registers would cost the plain selection a wave per SIMD)
__global__ __launch_bounds__(64) void k_select_bf16_gate(SelectLaunch p) { select_body<ActBF16, true>(p); }
__global__ __launch_bounds__(64) void k_select_f32(SelectLaunch p) { select_body<ActF32>(p); }

// A decode call over a device-LRU pool: wave t selects the experts of token t
// (softmax, top-k, renormalised scores, as select_body), then the block
// applies the LRU assign to the routed ids, tokens in order and slots in rank
// order (vm_lru.h).
static_assert(64 * kMaxExpertsPerLane <= kLruMaxExperts, "routed ids must fit the LRU's LDS map");

template <class A, int P>
__global__ __launch_bounds__(kLruThreads) void k_select_lru(SelectLaunch p, LruLaunch l) {
  __shared__ typename Cand<A>::T s_cands[kLruWaves][kMaxCand];
  __shared__ int32_t s_routed[kLruMaxRouted];
  __shared__ LruShared sh;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  LruRegs<P> r;
  lru_begin(l, sh, r);  // independent of the routing: in flight during the selection
  if (wave < p.tokens) {
    const uint32_t t = wave;
    GateKeys<A> g;
    float lg[kMaxExpertsPerLane];
    load_logits(p.logits + static_cast<size_t>(t) * p.experts, p.experts, lane, lg);
    softmax_keys<A>(lg, p.experts, lane, g);
    uint32_t e;
    float score;
    rank_selection<A>(g, p.top_k, p.blend, lane, s_cands[wave], e, score);
    if (lane < p.top_k) {
      const size_t o = static_cast<size_t>(t) * p.top_k + lane;
      p.inds[o] = static_cast<int32_t>(e);
      A::store(p.scores, o, score);
      s_routed[o] = static_cast<int32_t>(e);
    }
  }
  lru_owners(l, r);
  lds_barrier();
  lru_assign(l, s_routed, sh, r);
}

// -------------------------------------------------------------- front -----

// Blocks [0, router_blocks): router rows, one per wave, for the kFrontTokens
// tokens of grid row y; the blocks after them: the shared gate, one wave per
// token of that row.
template <class A, int CH>
__global__ __launch_bounds__(kFrontW * 64) void k_front(FrontLaunch p, uint32_t router_blocks) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  const uint32_t t_begin = blockIdx.y * kFrontTokens;
  const uint32_t t_end = min(p.tokens, t_begin + kFrontTokens);
  if (blockIdx.x >= router_blocks) {
    const uint32_t t = t_begin + (blockIdx.x - router_blocks) * kFrontW + wave;
    if (t < t_end) shared_gate_token<A>(p, t, lane);
  } else {
    const uint32_t row = blockIdx.x * kFrontW + wave;
    if (row < p.experts) {
      if (t_end - t_begin == 1) router_row<A, CH, 1>(p, row, lane, t_begin, t_end);
      else router_row<A, CH, kFrontUnroll>(p, row, lane, t_begin, t_end);
    }
  }
  if (p.trace != nullptr && threadIdx.x == 0) {
    tr.mark(1);
    tr.t[2] = tr.t[3] = tr.t[4] = tr.t[1];
    tr.write(p.trace, 1, blockIdx.y * gridDim.x + blockIdx.x);
  }
}

// ------------------------------------------------------------- gate/up ----

// SwiGLU of one row and the optional raw gate/up outputs.
template <class A>
__device__ __forceinline__ void gateup_store(const GateUpLaunch& p, uint32_t t, uint32_t j, uint32_t S, bool routed,
                                             bool ok, uint32_t row, float g, float u) {
  if (row >= p.inter) return;
  const float gv = A::round(g);
  const float uv = A::round(u);
  A::store(p.act, (static_cast<size_t>(t) * S + j) * p.inter + row, ok ? swiglu_act<A>(gv, uv) : 0.0f);
  if (routed) {
    const size_t o = (static_cast<size_t>(t) * p.slots + j) * p.inter + row;
    if (p.gate_out != nullptr) A::store(p.gate_out, o, gv);
    if (p.up_out != nullptr) A::store(p.up_out, o, uv);
  }
}

// LPR lanes per row (one 32-input group per lane and iteration, GI
// iterations), U rows per lane group; a block covers RPB = (64/LPR)*U*4 rows.
template <class A, int LPR, int GI, int U>
__global__ __launch_bounds__(kGuBlock) void k_gateup(GateUpLaunch p) {
  constexpr int RPI = 64 / LPR;
  constexpr int RPW = RPI * U;
  constexpr int RPB = RPW * kGuWaves;
  // every wave runs the selection itself (its own candidate list), so no
  // barrier stands between the selection and the weight loads
  __shared__ typename Cand<A>::T s_cands[kGuWaves][kMaxCand];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  typename Cand<A>::T* s_cand = s_cands[wave];
  const uint32_t lr = lane % LPR;
  const uint32_t rw = lane / LPR;
  const uint32_t pair = blockIdx.y;
  const uint32_t routed_pairs = p.tokens * p.slots;
  const bool shared_pair = pair >= routed_pairs;
  const uint32_t t = shared_pair ? pair - routed_pairs : pair / p.slots;
  const uint32_t j = shared_pair ? p.slots : pair % p.slots;
  const uint32_t S = p.slots + p.has_shared;
  const uint32_t H = p.hidden, I = p.inter, G = H / kGroup;
  uint32_t E = p.experts;
  const bool select = !shared_pair && p.logits != nullptr;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  // the arguments used after the selection, held in SGPRs from here on (the
  // stream view serves split-phase routes only and is read where it is used)
  PoolDev pool = p.pool;
  const PoolDev& stream = p.stream;
  keep_view<0, 6>(pool);
  ProjPtrs gate = p.gate, up = p.up;
  keep_proj(gate);
  keep_proj(up);
  VM_KEEP(E);
  VM_PIN(p.act);

  // 1. loads: the selection's logits and slot-table entries first, then this
  //    lane's activation groups
  // wave 0 selects for the block (the same pair for every wave) and hands the
  // route word over through LDS: the selection is VALU-bound, so doing it in
  // every wave only crowded the SIMDs
  __shared__ uint32_t s_word;
  const bool chooser = select && wave == 0;
  float lg[kMaxExpertsPerLane];
  int32_t tab[kMaxExpertsPerLane];
  if (chooser) {
    load_logits(p.logits + static_cast<size_t>(t) * E, E, lane, lg);
    if (p.slot_table != nullptr) {
#pragma unroll
      for (int m = 0; m < kMaxExpertsPerLane; ++m) tab[m] = p.slot_table[min(lane + 64u * m, E - 1)];
    }
  }
  asm volatile("" ::: "memory");
  GroupAct<A> xa[GI];
#pragma unroll
  for (int it = 0; it < GI; ++it) {
    const uint32_t g = lr + it * LPR;
    const bool live = g < G;
    xa[it].fetch(live ? p.x : g_zero_page, live ? static_cast<size_t>(t) * H + g * kGroup : 0);
  }

  // 2. the route word of this pair
  GateKeys<A> keys;
  uint32_t word = 0;
  if (select) {
    if (chooser) {
      softmax_keys<A>(lg, E, lane, keys);
      if (p.trace != nullptr) tr.mark(5);
      const uint32_t e = select_rank<A>(keys, p.slots, j, lane, s_cand);
      word = e;
      if (p.slot_table != nullptr) {
        const uint32_t m_e = e >> 6, l_e = e & 63u;
        int32_t slot = -1;
#pragma unroll
        for (int m = 0; m < kMaxExpertsPerLane; ++m)
          if (m == static_cast<int>(m_e)) slot = __builtin_amdgcn_readlane(tab[m], l_e);
        word = route_word(slot);
      }
      if (lane == 0) s_word = word;
      if (p.trace != nullptr) tr.mark(6);
    }
    lds_barrier();
    word = s_word;
  } else if (!shared_pair) {
    word = p.routes[t * p.slots + j];
  }

  ProjPtrs gp{}, upp{};
  bool ok = true;
  if (shared_pair) {
    gp = p.shared_gate;
    upp = p.shared_up;
  } else {
    uint32_t index = 0;
    const int kind = resolve_word(word, select ? nullptr : p.slot_table, E, pool, &stream,
                                  gate.w != nullptr && up.w != nullptr, index);
    ok = kind != kSrcNone;
    source_proj(kind, index, pool, &stream, gate, 0, I, H, gp);
    source_proj(kind, index, pool, &stream, up, 1, I, H, upp);
  }
  if (!ok && tid == 0 && blockIdx.x == 0) flag(p.status, 1u);
  if (p.trace != nullptr) tr.mark(1);

  // 3. stream the gate and up rows
  const uint32_t row_base = blockIdx.x * RPB + wave * RPW + rw;
  const uint32_t* zw = reinterpret_cast<const uint32_t*>(g_zero_page) + lr * kWordsPerGroup;
  const uint16_t* zm = reinterpret_cast<const uint16_t*>(g_zero_page) + lr;
  uint4 wg[U][GI], wu[U][GI];
  uint32_t sg[U][GI], bg[U][GI], su[U][GI], bu[U][GI];
  const size_t row_words = H / 8;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t row = row_base + u * RPI;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      const uint32_t g = lr + it * LPR;
      const bool live = ok && row < I && g < G;
      const size_t wo = static_cast<size_t>(row) * row_words + g * kWordsPerGroup;
      const size_t mo = static_cast<size_t>(row) * G + g;
      wg[u][it] = ldg16(live ? gp.w + wo : zw);
      wu[u][it] = ldg16(live ? upp.w + wo : zw);
      sg[u][it] = ldg_u16(live ? gp.s + mo : zm);
      bg[u][it] = ldg_u16(live ? gp.b + mo : zm);
      su[u][it] = ldg_u16(live ? upp.s + mo : zm);
      bu[u][it] = ldg_u16(live ? upp.b + mo : zm);
    }
  }

  // 4. one block per token publishes the ordered selection for the down kernel
  if (select && blockIdx.x == 0 && j == 0 && wave == 0) {
    uint32_t e;
    float score;
    rank_selection<A>(keys, p.slots, p.blend, lane, s_cand, e, score);
    if (lane < p.slots) {
      const size_t o = static_cast<size_t>(t) * p.slots + lane;
      if (p.inds_out != nullptr) p.inds_out[o] = static_cast<int32_t>(e);
      if (p.scores_out != nullptr) A::store(p.scores_out, o, score);
      if (p.words_out != nullptr) p.words_out[o] = p.slot_table != nullptr ? route_word(p.slot_table[e]) : e;
    }
  }

  // 5. group dots, row sums, SwiGLU
#pragma unroll
  for (int it = 0; it < GI; ++it) xa[it].prepare();
  float gs[U], us[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      ag += xa[it].apply(wg[u][it], bf16_to_f32(sg[u][it]), bf16_to_f32(bg[u][it]));
      au += xa[it].apply(wu[u][it], bf16_to_f32(su[u][it]), bf16_to_f32(bu[u][it]));
    }
    gs[u] = group_sum<LPR>(ag);
    us[u] = group_sum<LPR>(au);
    if (u == 0 && p.trace != nullptr) tr.mark(2);
  }
  if (p.trace != nullptr) tr.mark(3);
  if constexpr (LPR == 64) {
    // the U row sums sit in lane 63: lane u takes row u
    float gv = 0.0f, uv = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gs[u]), 63));
      const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, us[u]), 63));
      if (lane == static_cast<uint32_t>(u)) {
        gv = a;
        uv = b;
      }
    }
    if (lane < static_cast<uint32_t>(U)) gateup_store<A>(p, t, j, S, !shared_pair, ok, row_base + lane, gv, uv);
  } else {
    if (lr == LPR - 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) gateup_store<A>(p, t, j, S, !shared_pair, ok, row_base + u * RPI, gs[u], us[u]);
    }
  }
  if (p.trace != nullptr && tid == 0) {
    tr.mark(4);
    tr.write(p.trace, select ? 2 : 3, blockIdx.y * gridDim.x + blockIdx.x);
  }
}

// ----------------------------------------------------------------- down ---

constexpr int kDownMaxSlots = 12;                         // MAX_TOP_K (10) + shared, rounded up
#ifndef VM_DOWN_WAVES
#define VM_DOWN_WAVES 12
#endif
constexpr int kDownWaves = VM_DOWN_WAVES;                  // waves per down block
constexpr int kDownBlock = kDownWaves * 64;
constexpr int kDownSlotsPerWave = (kDownMaxSlots + kDownWaves - 1) / kDownWaves;  // wave w owns slots w + kDownWaves i
constexpr int kDownQuads = VM_DOWN_QUADS;                 // row groups of 64/LPR rows per block

// LPR = I/32 lanes per row (one group each); a block covers RB rows of all
// slots of one token.
// INJ: the combined rows are also injected into residual streams (p.inject);
// a separate instance, so the plain kernel carries none of its loads.
template <class A, int LPR, bool INJ>
__global__ __launch_bounds__(kDownBlock) void k_down(DownLaunch p) {
  constexpr int RPI = 64 / LPR;
  constexpr int RB = RPI * kDownQuads;
  __shared__ float s_part[kDownMaxSlots * RB];
  __shared__ float s_scores[kDownMaxSlots];
  __shared__ float s_shared[RB];
  __shared__ float s_sig;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t lr = lane % LPR;
  const uint32_t rw = lane / LPR;
  const uint32_t t = blockIdx.y;
  const uint32_t K = p.slots;
  const uint32_t S = K + p.has_shared;
  const uint32_t H = p.hidden, I = p.inter, G = I / kGroup;
  const uint32_t row0 = blockIdx.x * RB;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  PoolDev pool = p.pool;
  const PoolDev& stream = p.stream;
  keep_view<6, 3>(pool);
  ProjPtrs down = p.down, shared_down = p.shared_down;
  keep_proj(down);
  keep_proj(shared_down);
  uint32_t E = p.experts;
  VM_KEEP(E);
  VM_PIN(p.act);

  // 1. loads: the route words first (lane k < K reads slot k), then this
  //    wave's activation groups (slot wave + 4 i, group lr)
  const uint32_t route = ldg_u32(p.routes + static_cast<size_t>(t) * K + min(lane, K - 1));
  asm volatile("" ::: "memory");
  GroupAct<A> xa[kDownSlotsPerWave];
#pragma unroll
  for (int i = 0; i < kDownSlotsPerWave; ++i) {
    const uint32_t slot = wave + kDownWaves * i;
    const bool live = slot < S && lr < G;
    xa[i].fetch(live ? p.act : g_zero_page, live ? (static_cast<size_t>(t) * S + slot) * I + lr * kGroup : 0);
  }

  // epilogue operands as raw bits: loaded now, converted into LDS after the
  // weight loads are issued, so no load waits in front of those
  const bool combine = p.scores != nullptr;
  const uint32_t er = tid - 64;  // wave 1 fetches the shared term of the tile
  const void* sh_src = p.shared_y != nullptr ? p.shared_y : p.shared;
  const bool take_score = combine && tid < K;
  const bool take_shared = combine && tid >= 64 && er < RB && row0 + er < H && sh_src != nullptr;
  const void* sig_src = p.has_shared ? p.shared_sig : p.shared != nullptr ? p.shared_gate : nullptr;
  const bool take_sig = combine && tid == 128 && sig_src != nullptr;
  uint32_t r_score = 0, r_shared = 0, r_sig = 0;
  if (take_score) {
    const size_t o = static_cast<size_t>(t) * K + tid;
    r_score = p.score_dtype == 0 ? ldg_u16(static_cast<const uint16_t*>(p.scores) + o)
                                 : ldg_u32(static_cast<const uint32_t*>(p.scores) + o);
  }
  if (take_shared) r_shared = A::load_bits(sh_src, static_cast<size_t>(t) * H + row0 + er);
  if (take_sig) r_sig = A::load_bits(sig_src, t);
  // the streams this thread's combined row is injected into, and their weights
  const Inject& inj = p.inject;
  const bool take_inject = INJ && combine && tid < RB && row0 + tid < H;
  constexpr int kStreams = INJ ? static_cast<int>(kMaxStreams) : 1;
  uint32_t r_hid[kStreams], r_iw[kStreams];
  if constexpr (INJ) {
#pragma unroll
    for (int j = 0; j < kStreams; ++j) {
      const bool live = take_inject && static_cast<uint32_t>(j) < inj.hc;
      r_hid[j] = live ? A::load_bits(inj.hidden, (static_cast<size_t>(t) * inj.hc + j) * H + row0 + tid) : 0u;
      r_iw[j] = live ? A::load_bits(inj.weights, static_cast<size_t>(t) * inj.hc + j) : 0u;
    }
  }

  // 2. lane k < K resolves slot k; the waves take their slots' pointers with
  //    readlane and issue their weight loads
  ProjPtrs mine{};
  uint32_t index = 0;
  const int kind = lane < K ? resolve_word(route, p.slot_table, E, pool, &stream, down.w != nullptr, index)
                            : kSrcNone;
  source_proj(kind, index, pool, &stream, down, 2, H, I, mine);
  const bool mine_ok = kind != kSrcNone;
  if (!mine_ok && lane < K && wave == 0 && blockIdx.x == 0) flag(p.status, 1u);
  const uint64_t ok_mask = __ballot(mine_ok);
  if (p.trace != nullptr) tr.mark(5);
  const uint32_t* zw = reinterpret_cast<const uint32_t*>(g_zero_page) + lr * kWordsPerGroup;
  const uint16_t* zm = reinterpret_cast<const uint16_t*>(g_zero_page) + lr;
  uint4 w[kDownSlotsPerWave][kDownQuads];
  uint32_t sc[kDownSlotsPerWave][kDownQuads], bi[kDownSlotsPerWave][kDownQuads];
  const size_t row_words = I / 8;
#pragma unroll
  for (int i = 0; i < kDownSlotsPerWave; ++i) {
    // no branch around the loads: slots past S load zeros, so the first use
    // of the data, not its load, waits
    const uint32_t slot = wave + kDownWaves * i;
    ProjPtrs dp = shared_down;
    bool ok = slot < S;
    if (slot < K) {
      ok = (ok_mask >> slot) & 1u;
      dp.w = reinterpret_cast<const uint32_t*>(readlane_u64(reinterpret_cast<uint64_t>(mine.w), slot));
      dp.s = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mine.s), slot));
      dp.b = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mine.b), slot));
    }
#pragma unroll
    for (int q = 0; q < kDownQuads; ++q) {
      const uint32_t row = row0 + q * RPI + rw;
      const bool live = ok && row < H && lr < G;
      const size_t mo = static_cast<size_t>(row) * G + lr;
      w[i][q] = ldg16(live ? dp.w + static_cast<size_t>(row) * row_words + lr * kWordsPerGroup : zw);
      sc[i][q] = ldg_u16(live ? dp.s + mo : zm);
      bi[i][q] = ldg_u16(live ? dp.b + mo : zm);
    }
  }
  if (p.trace != nullptr) tr.mark(6);

  // 3. epilogue operands into LDS
  if (take_score) s_scores[tid] = p.score_dtype == 0 ? bf16_to_f32(r_score) : __uint_as_float(r_score);
  if (take_shared) s_shared[er] = A::from_bits(r_shared);
  if (take_sig) s_sig = A::from_bits(r_sig);
  if (p.trace != nullptr) tr.mark(7);

  // 4. dot products and row sums into LDS
#pragma unroll
  for (int i = 0; i < kDownSlotsPerWave; ++i) {
    const uint32_t slot = wave + kDownWaves * i;
    if (slot >= S) break;  // wave-uniform
    xa[i].prepare();
#pragma unroll
    for (int q = 0; q < kDownQuads; ++q) {
      float v = xa[i].apply(w[i][q], bf16_to_f32(sc[i][q]), bf16_to_f32(bi[i][q]));
      v = group_sum<LPR>(v);
      if (lr == LPR - 1) s_part[slot * RB + q * RPI + rw] = v;
    }
    if (i == 0 && p.trace != nullptr) tr.mark(2);
  }
  if (p.trace != nullptr) tr.mark(3);
  __syncthreads();
  if (p.trace != nullptr) tr.mark(1);

  // 5. combine in slot order
  if (p.scores != nullptr) {
    if (tid < RB && row0 + tid < H) {
      const uint32_t r = tid;
      float combined = 0.0f;
      if (p.generic) {
        for (uint32_t k = 0; k < K; ++k)
          combined = __fadd_rn(combined, A::round(__fmul_rn(A::round(s_part[k * RB + r]), s_scores[k])));
      } else {
        for (uint32_t k = 0; k < K; ++k)
          combined = __fadd_rn(combined, __fmul_rn(A::round(s_part[k * RB + r]), s_scores[k]));
      }
      float y = A::round(combined);
      if (p.has_shared) {
        const float sh = A::round(s_part[K * RB + r]);
        y = A::round(__fadd_rn(y, A::round(__fmul_rn(s_sig, sh))));
      } else if (p.shared_y != nullptr) {
        y = A::round(__fadd_rn(y, s_shared[r]));
      } else if (p.shared != nullptr) {
        y = A::round(__fadd_rn(y, A::round(__fmul_rn(s_shared[r], s_sig))));
      }
      A::store(p.out, static_cast<size_t>(t) * H + row0 + r, y);
      if (INJ && take_inject) {
#pragma unroll
        for (int j = 0; j < kStreams; ++j) {
          if (static_cast<uint32_t>(j) >= inj.hc) break;
          const float v = A::round(__fadd_rn(A::from_bits(r_hid[j]), A::round(__fmul_rn(y, A::from_bits(r_iw[j])))));
          A::store(inj.out, (static_cast<size_t>(t) * inj.hc + j) * H + row0 + r, v);
        }
      }
    }
  } else {
    for (uint32_t idx = tid; idx < K * RB; idx += kDownBlock) {
      const uint32_t k = idx / RB, r = idx % RB;
      if (row0 + r < H) A::store(p.out, (static_cast<size_t>(t) * K + k) * H + row0 + r, A::round(s_part[k * RB + r]));
    }
  }
  if (p.trace != nullptr && tid == 0) {
    tr.mark(4);
    tr.write(p.trace, 4, blockIdx.y * gridDim.x + blockIdx.x);
  }
}

// ------------------------------------------------------ weighted combine --

template <class A>
__global__ __launch_bounds__(kBlock) void k_weighted_combine(const void* values, const void* scores, void* out,
                                                             uint32_t tokens, uint32_t slots, uint32_t hidden,
                                                             int score_dtype) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= static_cast<size_t>(tokens) * hidden) return;
  const uint32_t t = static_cast<uint32_t>(i / hidden), h = static_cast<uint32_t>(i % hidden);
  float acc = 0.0f;
  for (uint32_t k = 0; k < slots; ++k) {
    const float v = A::load(values, (static_cast<size_t>(t) * slots + k) * hidden + h);
    acc = __fadd_rn(acc, __fmul_rn(v, load_any(scores, static_cast<size_t>(t) * slots + k, score_dtype)));
  }
  A::store(out, i, A::round(acc));
}

// ------------------------------------------------------------ dispatch ----

uint32_t next_pow2(uint32_t v) {
  uint32_t r = 1;
  while (r < v) r <<= 1;
  return r;
}

// One kernel launch of a timing family; with timing on, the start/stop events
// ride on the dispatch itself.
template <class... KArgs, class... Args>
hipError_t launch(const char* family, void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream,
                  Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
  return hipGetLastError();
}

template <class A, int LPR, int GI, int U>
hipError_t gateup_go(const GateUpLaunch& p, hipStream_t stream) {
  constexpr int RPB = (64 / LPR) * U * kGuWaves;
  const uint32_t pairs = p.tokens * p.slots + (p.has_shared ? p.tokens : 0);
  dim3 grid((p.inter + RPB - 1) / RPB, pairs);
  GateUpLaunch q = p;
  q.trace = trace_reserve(grid.x * grid.y);
  return launch("gateup", k_gateup<A, LPR, GI, U>, grid, dim3(kGuBlock), stream, q);
}

template <class A>
hipError_t gateup_dispatch(const GateUpLaunch& p, hipStream_t stream) {
  const uint32_t G = p.hidden / kGroup;
  const uint32_t lpr = G >= 64 ? 64 : next_pow2(G);
  const uint32_t gi = (G + 63) / 64;
  switch (lpr) {
    case 1: return gateup_go<A, 1, 1, 1>(p, stream);
    case 2: return gateup_go<A, 2, 1, 1>(p, stream);
    case 4: return gateup_go<A, 4, 1, 1>(p, stream);
    case 8: return gateup_go<A, 8, 1, 1>(p, stream);
    case 16: return gateup_go<A, 16, 1, 2>(p, stream);
    case 32: return gateup_go<A, 32, 1, 2>(p, stream);
    default: break;
  }
  if (gi <= 1) return gateup_go<A, 64, 1, kGateupRowsPerLane>(p, stream);
  if (gi <= 2) return gateup_go<A, 64, 2, 2>(p, stream);
  return gateup_go<A, 64, 4, 1>(p, stream);
}

template <class A, int LPR>
hipError_t down_go(const DownLaunch& p, hipStream_t stream) {
  constexpr int RB = (64 / LPR) * kDownQuads;
  dim3 grid((p.hidden + RB - 1) / RB, p.tokens);
  DownLaunch q = p;
  q.trace = trace_reserve(grid.x * grid.y);
  if (p.inject.out != nullptr) return launch("down", k_down<A, LPR, true>, grid, dim3(kDownBlock), stream, q);
  return launch("down", k_down<A, LPR, false>, grid, dim3(kDownBlock), stream, q);
}

template <class A>
hipError_t down_dispatch(const DownLaunch& p, hipStream_t stream) {
  switch (next_pow2(p.inter / kGroup)) {
    case 1: return down_go<A, 1>(p, stream);
    case 2: return down_go<A, 2>(p, stream);
    case 4: return down_go<A, 4>(p, stream);
    case 8: return down_go<A, 8>(p, stream);
    case 16: return down_go<A, 16>(p, stream);
    case 32: return down_go<A, 32>(p, stream);
    default: return down_go<A, 64>(p, stream);
  }
}

template <class A>
hipError_t front_go(const FrontLaunch& p0, hipStream_t stream) {
  const uint32_t router_blocks = (p0.experts + kFrontW - 1) / kFrontW;
  const uint32_t row_tokens = p0.tokens < kFrontTokens ? p0.tokens : kFrontTokens;
  const uint32_t shared_blocks = p0.seg.w != nullptr ? (row_tokens + kFrontW - 1) / kFrontW : 0;
  const dim3 grid(router_blocks + shared_blocks, (p0.tokens + kFrontTokens - 1) / kFrontTokens), block(kFrontW * 64);
  FrontLaunch p = p0;
  p.trace = trace_reserve(grid.x * grid.y);
  const uint32_t chunks = (p.hidden / 8 + 63) / 64;
  if (chunks <= 1) return launch("router", k_front<A, 1>, grid, block, stream, p, router_blocks);
  if (chunks <= 2) return launch("router", k_front<A, 2>, grid, block, stream, p, router_blocks);
  if (chunks <= 4) return launch("router", k_front<A, 4>, grid, block, stream, p, router_blocks);
  if (chunks <= 8) return launch("router", k_front<A, 8>, grid, block, stream, p, router_blocks);
  return launch("router", k_front<A, 16>, grid, block, stream, p, router_blocks);
}

}  // namespace

bool gateup_supported(uint32_t hidden) {
  return hidden % kGroup == 0 && hidden > 0 && hidden / kGroup <= 256;
}

bool down_supported(uint32_t inter, uint32_t slots_total, int /*act_dtype*/) {
  if (inter % kGroup != 0 || inter == 0 || inter / kGroup > 64) return false;
  return slots_total > 0 && slots_total <= static_cast<uint32_t>(kDownMaxSlots);
}

hipError_t launch_front(const FrontLaunch& p, hipStream_t stream) {
  return p.act_dtype == 0 ? front_go<ActBF16>(p, stream) : front_go<ActF32>(p, stream);
}

template <int P>
hipError_t select_lru_go(const SelectLaunch& p, const LruLaunch& l, hipStream_t stream) {
  const dim3 grid(1), block(kLruThreads);
  return p.act_dtype == 0 ? launch("lru", k_select_lru<ActBF16, P>, grid, block, stream, p, l)
                          : launch("lru", k_select_lru<ActF32, P>, grid, block, stream, p, l);
}

hipError_t launch_select_lru(const SelectLaunch& p, const LruLaunch& l, hipStream_t stream) {
  // queue entries per thread, rounded up to the instantiated powers of two
  const uint32_t per = (l.order_len + kLruThreads - 1) / kLruThreads;
  static_assert(kLruSlotsPerThread == 32, "instances below cover 1..32 entries per thread");
  if (per <= 1) return select_lru_go<1>(p, l, stream);
  if (per <= 2) return select_lru_go<2>(p, l, stream);
  if (per <= 4) return select_lru_go<4>(p, l, stream);
  if (per <= 8) return select_lru_go<8>(p, l, stream);
  if (per <= 16) return select_lru_go<16>(p, l, stream);
  if (per <= 32) return select_lru_go<32>(p, l, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_select(const SelectLaunch& p, hipStream_t stream) {
  const dim3 grid(p.tokens), block(64);
  if (p.seg.w != nullptr) {
    if (p.act_dtype != 0) return hipErrorInvalidValue;
    return launch("select", k_select_bf16_gate, grid, block, stream, p);
  }
  return p.act_dtype == 0 ? launch("select", k_select_bf16, grid, block, stream, p)
                          : launch("select", k_select_f32, grid, block, stream, p);
}

hipError_t launch_gateup(const GateUpLaunch& p, hipStream_t stream) {
  return p.act_dtype == 0 ? gateup_dispatch<ActBF16>(p, stream) : gateup_dispatch<ActF32>(p, stream);
}

hipError_t launch_down(const DownLaunch& p, hipStream_t stream) {
  return p.act_dtype == 0 ? down_dispatch<ActBF16>(p, stream) : down_dispatch<ActF32>(p, stream);
}

hipError_t launch_weighted_combine(const void* values, const void* scores, void* out, uint32_t tokens,
                                   uint32_t slots, uint32_t hidden, int act_dtype, int score_dtype,
                                   hipStream_t stream) {
  const size_t n = static_cast<size_t>(tokens) * hidden;
  const dim3 grid(static_cast<uint32_t>((n + kBlock - 1) / kBlock)), block(kBlock);
  if (act_dtype == 0)
    return launch("combine", k_weighted_combine<ActBF16>, grid, block, stream, values, scores, out, tokens, slots,
                  hidden, score_dtype);
  return launch("combine", k_weighted_combine<ActF32>, grid, block, stream, values, scores, out, tokens, slots,
                hidden, score_dtype);
}

}  // namespace vm
