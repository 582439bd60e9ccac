// Decode of one token in two launches (gfx950, wave64).
//
//   k_fused_front    router logits (one row per wave, as k_front), the shared
//                    expert's gate/up + SwiGLU and its H -> 1 sigmoid gate,
//                    which do not depend on the routing, and the zeroing of
//                    the hand-off words of the experts kernel.
//   k_fused_experts  one block per CU.  Every wave selects the top-k from the
//                    logits (or takes the routes of the device LRU), resolves
//                    each expert's pool slot, and issues the loads of its
//                    gate/up rows and of its down rows at once: both are
//                    known as soon as the routing is, so the down weights
//                    stream while gate/up computes.  Each activation is
//                    published as a tagged word (1 << 16 | bf16) written
//                    through to memory (agent-scope store); every block then
//                    reads the activations of all routed experts into LDS,
//                    waiting (bounded) until each word carries the tag, and
//                    computes its tiles of down rows for every slot and the
//                    slot-order combine.
//
// The hand-off needs no counter, fence or L2 writeback: a word is read
// through to memory too, and it is valid exactly when its tag is set, since
// the front kernel zeroed every word before this launch began.  Producers
// never wait, and a block waits only after its own gate/up work is published,
// with one block per CU so the whole grid is resident.
//
// The arithmetic is the three-launch path's, operation for operation (the
// same group dots, DPP reduction trees, SwiGLU and combine order), so both
// give the same bits.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "vm_internal.h"
#include "vm_select.h"

// Both pipelines were measured slower than the three-launch default (18.4
// and 24.1 against 16.2 us per layer at hidden 2048 / inter 512 / 512 experts
// top-10 + shared), so the shipped library leaves them out; a build with
// -DVM_FUSED_PIPELINES=1 carries them for A/B measurement and their parity
// tests.  Without them the entry points below refuse every shape, and
// vm_decode_pipeline accepts mode 0 only.
#if VM_FUSED_PIPELINES

namespace vm {

namespace {

constexpr int kFrontWaves = 4;
constexpr int kFrontBlock = kFrontWaves * 64;
constexpr int kXWaves = 8;
constexpr int kXBlock = kXWaves * 64;
constexpr uint32_t kTagBit = 1u << 16;
constexpr uint64_t kPairTags = (1ull << 16) | (1ull << 48);
constexpr uint32_t kWaitLimit = 1u << 16;   // polls of one word before giving up (status bit 5)
constexpr uint32_t kStatusWait = 32u;

__device__ __forceinline__ void store_through(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t load_through(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ FrontLaunch front_args(const FusedLaunch& p) {
  FrontLaunch f{};
  f.x = p.x;
  f.weight = p.router;
  f.bias = p.router_bias;
  f.logits = p.logits;
  f.seg = p.sh_seg;
  f.shared_sig = p.sh_sig;
  f.tokens = 1;
  f.hidden = p.hidden;
  f.experts = p.experts;
  f.act_dtype = 0;
  return f;
}

// ------------------------------------------------------------- front ------
// Blocks [0, router_blocks): one router row per wave.  The next shared_blocks:
// RPG rows of the shared expert's gate and up per wave, SwiGLU into sh_act.
// The last block: the shared gate (wave 0).  Every thread first zeroes its
// share of the hand-off words.
template <int CH, int LG, int GI>
__global__ __launch_bounds__(kFrontBlock) void k_fused_front(FusedLaunch p, uint32_t router_blocks,
                                                              uint32_t shared_blocks) {
  constexpr int RPG = 64 / LG;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t b = blockIdx.x;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  const uint32_t words = p.act_tag != nullptr ? p.slots * p.inter : 0u;
  for (uint32_t i = b * kFrontBlock + threadIdx.x; i < words; i += gridDim.x * kFrontBlock) p.act_tag[tag_index(i)] = 0u;
  const FrontLaunch f = front_args(p);
  if (b < router_blocks) {
    const uint32_t row = b * kFrontWaves + wave;
    if (row < p.experts) router_row<ActBF16, CH, 1>(f, row, lane, 0, 1);
  } else if (b < router_blocks + shared_blocks) {
    const uint32_t H = p.hidden, G = H / kGroup, I = p.inter;
    const uint32_t lr = lane % LG, rw = lane / LG;
    const uint32_t row = ((b - router_blocks) * kFrontWaves + wave) * RPG + rw;
    const uint32_t* zw = reinterpret_cast<const uint32_t*>(g_zero_page) + lr * kWordsPerGroup;
    const uint16_t* zm = reinterpret_cast<const uint16_t*>(g_zero_page) + lr;
    GroupAct<ActBF16> xa[GI];
    uint4 wg[GI], wu[GI];
    uint32_t sg[GI], bg[GI], su[GI], bu[GI];
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      const uint32_t g = lr + it * LG;
      const bool gl = g < G;
      xa[it].fetch(gl ? static_cast<const void*>(p.x) : g_zero_page, gl ? g * kGroup : 0);
      const bool live = gl && row < I;
      const size_t wo = static_cast<size_t>(row) * (H / 8) + g * kWordsPerGroup;
      const size_t mo = static_cast<size_t>(row) * G + g;
      wg[it] = ldg16(live ? p.sh_gate.w + wo : zw);
      wu[it] = ldg16(live ? p.sh_up.w + wo : zw);
      sg[it] = ldg_u16(live ? p.sh_gate.s + mo : zm);
      bg[it] = ldg_u16(live ? p.sh_gate.b + mo : zm);
      su[it] = ldg_u16(live ? p.sh_up.s + mo : zm);
      bu[it] = ldg_u16(live ? p.sh_up.b + mo : zm);
    }
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      xa[it].prepare();
      ag += xa[it].apply(wg[it], bf16_to_f32(sg[it]), bf16_to_f32(bg[it]));
      au += xa[it].apply(wu[it], bf16_to_f32(su[it]), bf16_to_f32(bu[it]));
    }
    ag = group_sum<LG>(ag);
    au = group_sum<LG>(au);
    if (lr == LG - 1 && row < I)
      p.sh_act[row] = static_cast<uint16_t>(f32_to_bf16(swiglu_act<ActBF16>(round_bf16(ag), round_bf16(au))));
  } else if (wave == 0) {
    shared_gate_token<ActBF16>(f, 0, lane);
  }
  if (p.trace != nullptr && threadIdx.x == 0) {
    tr.mark(1);
    tr.t[2] = tr.t[3] = tr.t[4] = tr.t[1];
    tr.write(p.trace, 1, b);
  }
}

// ----------------------------------------------------------- experts ------
// Work of block b in a grid of NB blocks:
//   gate/up item i (RPG rows of one routed slot) for i = b + NB (w + 8u): wave w, u < kFusedMaxGateUp;
//   down tile t (RPD output rows, every slot) for t = b + NB q; item d = q S + s of
//   the block (slot s) on wave d % 8, position d / 8 < kFusedMaxDown.
// DOWN: the two-launch pipeline (hand-off and down rows here); otherwise the
// grid ends after gate/up, writing the activations and the route words for
// the down kernel of the three-launch pipeline.
template <int LG, int GI, int LD, bool DOWN>
__global__ __launch_bounds__(kXBlock) void k_fused_experts(FusedLaunch p) {
  constexpr int RPG = 64 / LG;
  constexpr int RPD = 64 / LD;
  constexpr int UG = kFusedMaxGateUp;
  constexpr int UD = kFusedMaxDown;
  using C = Cand<ActBF16>;
  __shared__ C::T s_cands[kXWaves][kMaxCand];
  __shared__ __align__(16) uint32_t s_act[kFusedMaxSlots * kFusedMaxInter / 2];  // bf16 pairs, slot-major
  __shared__ float s_part[kXWaves * UD][RPD];
  __shared__ float s_scores[kFusedMaxSlots];
  __shared__ float s_sig;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6)));
  const uint32_t b = blockIdx.x;
  const uint32_t NB = gridDim.x;
  const uint32_t K = p.slots, S = K + p.has_shared;
  const uint32_t H = p.hidden, I = p.inter, G = H / kGroup, GD = I / kGroup;
  uint32_t E = p.experts;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  PoolDev pool = p.pool;
  keep_view<0, 9>(pool);
  ProjPtrs gate = p.gate, up = p.up, down = p.down;
  keep_proj(gate);
  keep_proj(up);
  keep_proj(down);
  VM_KEEP(E);

  // 1. loads: the routing inputs first, then this lane's activation groups
  const bool select = p.routes == nullptr;
  float lg[kMaxExpertsPerLane];
  int32_t tab[kMaxExpertsPerLane];
  uint32_t r_route = 0, r_score = 0;
  if (select) {
    load_logits(p.logits, E, lane, lg);
    if (p.slot_table != nullptr) {
#pragma unroll
      for (int m = 0; m < kMaxExpertsPerLane; ++m) tab[m] = p.slot_table[min(lane + 64u * m, E - 1)];
    }
  } else {
    r_route = ldg_u32(p.routes + min(lane, K - 1));
    r_score = ldg_u16(p.route_scores + min(lane, K - 1));
  }
  const uint32_t r_sig = p.has_shared ? ldg_u16(p.sh_sig) : 0u;
  asm volatile("" ::: "memory");
  const uint32_t lr = lane % LG, rw = lane / LG;
  GroupAct<ActBF16> xa[GI];
#pragma unroll
  for (int it = 0; it < GI; ++it) {
    const uint32_t g = lr + it * LG;
    const bool live = g < G;
    xa[it].fetch(live ? static_cast<const void*>(p.x) : g_zero_page, live ? g * kGroup : 0);
  }

  // 2. the routing: lane k < K holds the expert of rank k and its pool slot
  C::T* cand = s_cands[wave];
  C::T top = 0;
  uint32_t e_k = 0;
  int32_t slot_k = -1;
  if (select) {
    GateKeys<ActBF16> keys;
    softmax_keys<ActBF16>(lg, E, lane, keys);
    top = rank_order<ActBF16>(keys, K, lane, cand);
    e_k = lane < K ? C::expert(top) : 0u;
    if (p.slot_table != nullptr) {
      // the table entry of e_k sits in lane e_k % 64, register e_k / 64
      const int src = static_cast<int>((e_k & 63u) << 2);
      const uint32_t m_e = e_k >> 6;
#pragma unroll
      for (int m = 0; m < kMaxExpertsPerLane; ++m) {
        const int32_t v = __builtin_amdgcn_ds_bpermute(src, tab[m]);
        if (m_e == static_cast<uint32_t>(m)) slot_k = v;
      }
    }
  } else {
    e_k = r_route;
    if (p.slot_table != nullptr) slot_k = p.slot_table[min(e_k, E - 1)];
  }
  if (p.trace != nullptr) tr.mark(5);
  // lane k's gate, up and down parts
  ProjPtrs mg{}, mu{}, md{};
  bool mine_ok = false;
  if (lane < K) {
    if (p.slot_table != nullptr) {
      mine_ok = e_k < E && slot_k >= 0 && static_cast<uint32_t>(slot_k) < pool.records;
      if (mine_ok) {
        record_parts(pool, static_cast<uint32_t>(slot_k), 0, mg);
        record_parts(pool, static_cast<uint32_t>(slot_k), 1, mu);
        record_parts(pool, static_cast<uint32_t>(slot_k), 2, md);
      }
    } else {
      mine_ok = e_k < E && gate.w != nullptr;
      if (mine_ok) {
        source_proj(kSrcDense, e_k, pool, nullptr, gate, 0, I, H, mg);
        source_proj(kSrcDense, e_k, pool, nullptr, up, 1, I, H, mu);
        source_proj(kSrcDense, e_k, pool, nullptr, down, 2, H, I, md);
      }
    }
  }
  const uint64_t ok_mask = __ballot(mine_ok);
  if (lane < K && !mine_ok && wave == 0 && b == 0 && p.status != nullptr) atomicOr(p.status, 1u);

  // 3. gate/up loads of this wave's items
  const uint32_t* zw = reinterpret_cast<const uint32_t*>(g_zero_page) + (lane % 8) * kWordsPerGroup;
  const uint16_t* zm = reinterpret_cast<const uint16_t*>(g_zero_page) + lane;
  const uint32_t per_slot = I / RPG;
  uint4 wg[UG][GI], wu[UG][GI];
  uint32_t sg[UG][GI], bg[UG][GI], su[UG][GI], bu[UG][GI];
  uint32_t gu_k[UG], gu_row[UG];
  bool gu_item[UG], gu_ok[UG];
#pragma unroll
  for (int u = 0; u < UG; ++u) {
    const uint32_t i = b + NB * (wave + kXWaves * u);
    gu_item[u] = i < p.gu_items;
    const uint32_t k = gu_item[u] ? i / per_slot : 0u;
    gu_k[u] = k;
    gu_row[u] = (gu_item[u] ? (i % per_slot) * RPG : 0u) + rw;
    gu_ok[u] = gu_item[u] && ((ok_mask >> k) & 1u);
    ProjPtrs gp, upp;
    gp.w = reinterpret_cast<const uint32_t*>(readlane_u64(reinterpret_cast<uint64_t>(mg.w), k));
    gp.s = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mg.s), k));
    gp.b = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mg.b), k));
    upp.w = reinterpret_cast<const uint32_t*>(readlane_u64(reinterpret_cast<uint64_t>(mu.w), k));
    upp.s = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mu.s), k));
    upp.b = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mu.b), k));
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      const uint32_t g = lr + it * LG;
      const uint32_t row = gu_row[u];
      const bool live = gu_ok[u] && row < I && g < G;
      const size_t wo = static_cast<size_t>(row) * (H / 8) + g * kWordsPerGroup;
      const size_t mo = static_cast<size_t>(row) * G + g;
      wg[u][it] = ldg16(live ? gp.w + wo : zw);
      wu[u][it] = ldg16(live ? upp.w + wo : zw);
      sg[u][it] = ldg_u16(live ? gp.s + mo : zm);
      bg[u][it] = ldg_u16(live ? gp.b + mo : zm);
      su[u][it] = ldg_u16(live ? upp.s + mo : zm);
      bu[u][it] = ldg_u16(live ? upp.b + mo : zm);
    }
  }

  // 4. down loads of this wave's items (slot S-1 is the shared expert)
  const uint32_t lrd = lane % LD, rwd = lane / LD;
  const uint32_t tiles_b = DOWN && b < p.dn_tiles ? (p.dn_tiles - b + NB - 1) / NB : 0u;
  uint4 wd[UD];
  uint32_t sd[UD], bd[UD];
  bool dn_item[UD];
#pragma unroll
  for (int u = 0; u < (DOWN ? UD : 0); ++u) {
    const uint32_t d = wave + kXWaves * u;
    const uint32_t q = d / S, s = d % S;
    dn_item[u] = q < tiles_b;
    const uint32_t row = (b + NB * q) * RPD + rwd;
    const uint32_t ks = s < K ? s : 0u;
    ProjPtrs dp = p.sh_down;
    bool ok = s >= K;
    if (s < K) {   // wave-uniform
      ok = (ok_mask >> ks) & 1u;
      dp.w = reinterpret_cast<const uint32_t*>(readlane_u64(reinterpret_cast<uint64_t>(md.w), ks));
      dp.s = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(md.s), ks));
      dp.b = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(md.b), ks));
    }
    const bool live = dn_item[u] && ok && row < H && lrd < GD;
    const size_t mo = static_cast<size_t>(row) * GD + lrd;
    wd[u] = ldg16(live ? dp.w + static_cast<size_t>(row) * (I / 8) + lrd * kWordsPerGroup : zw);
    sd[u] = ldg_u16(live ? dp.s + mo : zm);
    bd[u] = ldg_u16(live ? dp.b + mo : zm);
  }
  if (p.trace != nullptr) tr.mark(6);

  // 5. the scores (wave 0), published by block 0
  if (wave == 0) {
    const float sc = select ? score_of_order<ActBF16>(cand, top, K, p.blend, lane) : bf16_to_f32(r_score);
    if (lane < K) s_scores[lane] = sc;
    if (lane == 0) s_sig = bf16_to_f32(r_sig);
    if (b == 0 && lane < K) {
      if (p.inds_out != nullptr) p.inds_out[lane] = static_cast<int32_t>(e_k);
      if (p.scores_out != nullptr) p.scores_out[lane] = static_cast<uint16_t>(f32_to_bf16(sc));
      if (!DOWN && p.words_out != nullptr)
        p.words_out[lane] = p.slot_table != nullptr ? route_word(slot_k) : e_k;
    }
  }

  // 6. gate/up dots, SwiGLU, activations published with their tag
#pragma unroll
  for (int it = 0; it < GI; ++it) xa[it].prepare();
#pragma unroll
  for (int u = 0; u < UG; ++u) {
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      ag += xa[it].apply(wg[u][it], bf16_to_f32(sg[u][it]), bf16_to_f32(bg[u][it]));
      au += xa[it].apply(wu[u][it], bf16_to_f32(su[u][it]), bf16_to_f32(bu[u][it]));
    }
    ag = group_sum<LG>(ag);
    au = group_sum<LG>(au);
    if (lr == LG - 1 && gu_item[u] && gu_row[u] < I) {
      const float a = gu_ok[u] ? swiglu_act<ActBF16>(round_bf16(ag), round_bf16(au)) : 0.0f;
      if constexpr (DOWN)
        store_through(p.act_tag + tag_index(gu_k[u] * I + gu_row[u]), kTagBit | f32_to_bf16(a));
      else
        p.act[static_cast<size_t>(gu_k[u]) * I + gu_row[u]] = static_cast<uint16_t>(f32_to_bf16(a));
    }
  }
  if (p.trace != nullptr) tr.mark(2);
  if constexpr (!DOWN) {
    if (p.trace != nullptr && tid == 0) {
      tr.t[3] = tr.t[1] = tr.t[2];
      tr.mark(4);
      tr.write(p.trace, 6, b);
    }
    return;
  }

  // 7. every slot's activations into LDS: the routed ones once their tag is
  //    set, the shared expert's from the front kernel
  if (tiles_b > 0) {
    const uint32_t pairs = K * I / 2;
    const uint32_t* words = p.act_tag;
    constexpr int kBatch = 8;
    for (uint32_t j0 = tid; j0 < pairs; j0 += kXBlock * kBatch) {
      // every word of the batch is read together; the ones whose tag is not
      // set yet are read again together, one round trip per round
      uint64_t v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const uint32_t j = j0 + i * kXBlock;
        v[i] = j < pairs ? load_through(reinterpret_cast<const uint64_t*>(words + tag_index(2 * j))) : kPairTags;
      }
      for (uint32_t polls = 0;; ++polls) {
        bool ready = true;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) ready = ready && (v[i] & kPairTags) == kPairTags;
        if (ready) break;
        if (polls == kWaitLimit) {
          if (p.status != nullptr) atomicOr(p.status, kStatusWait);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const uint32_t j = j0 + i * kXBlock;
          if ((v[i] & kPairTags) != kPairTags)
            v[i] = load_through(reinterpret_cast<const uint64_t*>(words + tag_index(2 * j)));
        }
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const uint32_t j = j0 + i * kXBlock;
        if (j < pairs) s_act[j] = static_cast<uint32_t>(v[i] & 0xffffu) | (static_cast<uint32_t>(v[i] >> 32) << 16);
      }
    }
    if (p.has_shared) {
      const uint32_t* sh = reinterpret_cast<const uint32_t*>(p.sh_act);
      for (uint32_t j = tid; j < I / 2; j += kXBlock) s_act[pairs + j] = ldg_u32(sh + j);
    }
  }
  __syncthreads();
  if (p.trace != nullptr) tr.mark(3);

  // 8. down dots of this wave's items into s_part
#pragma unroll
  for (int u = 0; u < UD; ++u) {
    if (!dn_item[u]) break;   // wave-uniform; items run in order
    const uint32_t d = wave + kXWaves * u;
    const uint32_t s = d % S;
    GroupAct<ActBF16> ya;
    if (lrd < GD) {
      const uint4* src = reinterpret_cast<const uint4*>(s_act + (s * I + lrd * kGroup) / 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 r = src[q];
        ya.xp[4 * q] = r.x; ya.xp[4 * q + 1] = r.y; ya.xp[4 * q + 2] = r.z; ya.xp[4 * q + 3] = r.w;
      }
    } else {
      ya.zero();
    }
    ya.prepare();
    float v = ya.apply(wd[u], bf16_to_f32(sd[u]), bf16_to_f32(bd[u]));
    v = group_sum<LD>(v);
    if (lrd == LD - 1) s_part[d][rwd] = v;
  }
  __syncthreads();
  if (p.trace != nullptr) tr.mark(1);

  // 9. slot-order combine of each row of this block's tiles
  if (tid < tiles_b * RPD) {
    const uint32_t q = tid / RPD, r = tid % RPD;
    const uint32_t row = (b + NB * q) * RPD + r;
    if (row < H) {
      float combined = 0.0f;
      if (p.generic) {
        for (uint32_t k = 0; k < K; ++k)
          combined = __fadd_rn(combined, round_bf16(__fmul_rn(round_bf16(s_part[q * S + k][r]), s_scores[k])));
      } else {
        for (uint32_t k = 0; k < K; ++k)
          combined = __fadd_rn(combined, __fmul_rn(round_bf16(s_part[q * S + k][r]), s_scores[k]));
      }
      float y = round_bf16(combined);
      if (p.has_shared) {
        const float sh = round_bf16(s_part[q * S + K][r]);
        y = round_bf16(__fadd_rn(y, round_bf16(__fmul_rn(s_sig, sh))));
      }
      p.out[row] = static_cast<uint16_t>(f32_to_bf16(y));
      const Inject& inj = p.inject;
      if (inj.out != nullptr) {
        for (uint32_t j = 0; j < inj.hc; ++j) {
          const float hv = ActBF16::load(inj.hidden, static_cast<size_t>(j) * H + row);
          const float wv = ActBF16::load(inj.weights, j);
          ActBF16::store(inj.out, static_cast<size_t>(j) * H + row,
                         round_bf16(__fadd_rn(hv, round_bf16(__fmul_rn(y, wv)))));
        }
      }
    }
  }
  if (p.trace != nullptr && tid == 0) {
    tr.mark(4);
    tr.write(p.trace, 5, b);
  }
}

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

uint32_t pow2_at_least(uint32_t v) {
  uint32_t r = 1;
  while (r < v) r <<= 1;
  return r;
}

// (lanes per gate/up row, groups per lane) of a hidden size; (0, 0) when the
// fused kernels have no instance for it
void gateup_shape(uint32_t hidden, uint32_t& lg, uint32_t& gi) {
  const uint32_t G = hidden / kGroup;
  lg = G >= 64 ? 64 : pow2_at_least(G);
  gi = (G + 63) / 64;
  // hidden sizes above 4096 (four groups per lane) would spill: the
  // three-launch path serves them
  if (lg < 8 || gi > 2) lg = gi = 0;
}

template <int LG, int GI>
hipError_t front_go(const FusedLaunch& p0, hipStream_t stream) {
  constexpr int CH = LG == 64 ? 4 * GI : (LG == 32 ? 2 : 1);
  constexpr int RPG = 64 / LG;
  const uint32_t router_blocks = (p0.experts + kFrontWaves - 1) / kFrontWaves;
  const uint32_t shared_blocks = p0.has_shared ? (p0.inter / RPG + kFrontWaves - 1) / kFrontWaves : 0u;
  const uint32_t blocks = router_blocks + shared_blocks + (p0.has_shared ? 1u : 0u);
  FusedLaunch p = p0;
  p.trace = trace_reserve(blocks);
  return launch("router", k_fused_front<CH, LG, GI>, dim3(blocks), dim3(kFrontBlock), stream, p, router_blocks,
                shared_blocks);
}

template <int LG, int GI, int LD, bool DOWN>
hipError_t experts_go(const FusedLaunch& p0, uint32_t blocks, hipStream_t stream) {
  FusedLaunch p = p0;
  p.trace = trace_reserve(blocks);
  return launch(DOWN ? "experts" : "gateup", k_fused_experts<LG, GI, LD, DOWN>, dim3(blocks), dim3(kXBlock),
                stream, p);
}

template <int LG, int GI>
hipError_t experts_by_down(const FusedLaunch& p, uint32_t blocks, bool down, hipStream_t stream) {
  if (!down) return experts_go<LG, GI, 4, false>(p, blocks, stream);
  switch (pow2_at_least(p.inter / kGroup)) {
    case 4: return experts_go<LG, GI, 4, true>(p, blocks, stream);
    case 8: return experts_go<LG, GI, 8, true>(p, blocks, stream);
    case 16: return experts_go<LG, GI, 16, true>(p, blocks, stream);
    case 32: return experts_go<LG, GI, 32, true>(p, blocks, stream);
    case 64: return experts_go<LG, GI, 64, true>(p, blocks, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool fused_plan(uint32_t hidden, uint32_t inter, uint32_t slots, uint32_t has_shared, uint32_t experts,
                uint32_t blocks, FusedLaunch& p) {
  uint32_t lg, gi;
  gateup_shape(hidden, lg, gi);
  const uint32_t GD = inter / kGroup;
  const uint32_t ld = pow2_at_least(GD);
  if (lg == 0 || ld < 4 || ld > 64 || inter > kFusedMaxInter || slots == 0 || experts == 0 ||
      experts > 64u * kMaxExpertsPerLane || slots + has_shared > kFusedMaxSlots || blocks == 0)
    return false;
  const uint32_t rpg = 64 / lg, rpd = 64 / ld;
  if (inter % rpg != 0) return false;
  const uint32_t gu_items = slots * inter / rpg;
  const uint32_t dn_tiles = (hidden + rpd - 1) / rpd;
  const uint32_t waves = blocks * kXWaves;
  const uint32_t tiles_per_block = (dn_tiles + blocks - 1) / blocks;
  if ((gu_items + waves - 1) / waves > static_cast<uint32_t>(kFusedMaxGateUp)) return false;
  if ((slots + has_shared) * tiles_per_block > static_cast<uint32_t>(kXWaves * kFusedMaxDown)) return false;
  p.gu_items = gu_items;
  p.dn_tiles = dn_tiles;
  return true;
}

hipError_t launch_fused_front(const FusedLaunch& p, hipStream_t stream) {
  uint32_t lg, gi;
  gateup_shape(p.hidden, lg, gi);
  switch (lg * 8 + gi) {
    case 8 * 8 + 1: return front_go<8, 1>(p, stream);
    case 16 * 8 + 1: return front_go<16, 1>(p, stream);
    case 32 * 8 + 1: return front_go<32, 1>(p, stream);
    case 64 * 8 + 1: return front_go<64, 1>(p, stream);
    case 64 * 8 + 2: return front_go<64, 2>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fused_experts(const FusedLaunch& p, uint32_t blocks, bool down, hipStream_t stream) {
  uint32_t lg, gi;
  gateup_shape(p.hidden, lg, gi);
  switch (lg * 8 + gi) {
    case 8 * 8 + 1: return experts_by_down<8, 1>(p, blocks, down, stream);
    case 16 * 8 + 1: return experts_by_down<16, 1>(p, blocks, down, stream);
    case 32 * 8 + 1: return experts_by_down<32, 1>(p, blocks, down, stream);
    case 64 * 8 + 1: return experts_by_down<64, 1>(p, blocks, down, stream);
    case 64 * 8 + 2: return experts_by_down<64, 2>(p, blocks, down, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vm

#else  // VM_FUSED_PIPELINES

namespace vm {

bool fused_plan(uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, FusedLaunch&) { return false; }
hipError_t launch_fused_front(const FusedLaunch&, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_fused_experts(const FusedLaunch&, uint32_t, bool, hipStream_t) { return hipErrorInvalidValue; }

}  // namespace vm

#endif  // VM_FUSED_PIPELINES
