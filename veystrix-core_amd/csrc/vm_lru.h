// Device side of the expert pool's LRU (one block of kLruThreads threads).
//
// The reference's ExpertPool.assign (models/flashnext/expert_pool.py:123-159)
// on per-slot stamps: every slot carries a distinct stamp, free slots the
// smallest (in the order the reference's free list pops them).  The hits of a
// call get the next stamps in first-seen order; then the M misses take the M
// slots with the smallest remaining stamps, oldest first, and get the stamps
// after those: the OrderedDict's move_to_end / popitem(last=False) order.
//
// Victims without a sort: each thread keeps the stamps of its slots (slot
// tid + kLruThreads * i) in registers; every wave extracts the M smallest
// stamps of its slots by repeated wave minima (a lane rescans its registers
// only after giving up its minimum), and one wave merges the 16 sorted lists.
#pragma once

#include "vm_internal.h"

namespace vm {

constexpr int kLruWaves = kLruThreads / 64;
constexpr uint64_t kLruNoStamp = ~0ull;

struct LruShared {
  int32_t dexp[kLruMaxRouted];    // distinct ids in first-seen order
  int32_t dslot[kLruMaxRouted];   // their slots, -1 on a miss
  int32_t miss[kLruMaxRouted];    // missed ids in first-seen order
  uint64_t cand[kLruWaves][kLruMaxRouted];
  uint32_t cslot[kLruWaves][kLruMaxRouted];
  uint32_t ccount[kLruWaves];
  uint32_t victim[kLruMaxRouted];
  uint32_t hits, misses, valid;
};

__device__ __forceinline__ uint32_t lru_mbcnt(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Smallest of the thread's stamps above `floor` (kLruNoStamp if none) and its slot.
__device__ __forceinline__ uint64_t lru_next(const uint64_t (&st)[kLruSlotsPerThread], uint32_t first, uint32_t slots,
                                             uint64_t floor, uint32_t& slot) {
  uint64_t best = kLruNoStamp;
  slot = 0;
#pragma unroll
  for (int i = 0; i < kLruSlotsPerThread; ++i) {
    const uint32_t s = first + static_cast<uint32_t>(i) * kLruThreads;
    const uint64_t v = st[i];
    if (s < slots && v > floor && v < best) {
      best = v;
      slot = s;
    }
  }
  return best;
}

// assign() of the routed ids in `routed` (LDS, -1 = skipped) for one call.
// Every thread of the block must call it (it holds block barriers).
__device__ void lru_assign(const LruLaunch& p, const int32_t* routed, LruShared& sh) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t N = p.routed, E = p.experts, S = p.slots;
  const uint32_t keys = p.layers * E;
  int32_t* table = p.slot_table + static_cast<size_t>(p.layer) * E;
  const uint64_t base = p.counters[0];

  // 1. one wave: distinct ids in first-seen order, their slots, hits stamped
  if (wave == 0) {
    uint32_t nd = 0, valid = 0;
    for (uint32_t c = 0; c < N; c += 64) {
      const uint32_t i = c + lane;
      const int32_t e = i < N ? routed[i] : -1;
      bool first = e >= 0;
      for (uint32_t j = 0; j < i && first; ++j) first = routed[j] != e;
      valid += __popcll(__ballot(e >= 0));
      const uint64_t fm = __ballot(first);
      if (first) {
        const uint32_t d = nd + lru_mbcnt(fm);
        const int32_t slot = table[e];
        sh.dexp[d] = e;
        sh.dslot[d] = slot >= 0 && static_cast<uint32_t>(slot) < S ? slot : -1;
      }
      nd += __popcll(fm);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    uint32_t hits = 0, misses = 0;
    for (uint32_t c = 0; c < nd; c += 64) {
      const uint32_t d = c + lane;
      const int32_t slot = d < nd ? sh.dslot[d] : -1;
      const bool hit = d < nd && slot >= 0;
      const bool miss = d < nd && slot < 0;
      const uint64_t hm = __ballot(hit), mm = __ballot(miss);
      if (hit) p.slot_stamp[slot] = base + 1 + hits + lru_mbcnt(hm);  // move to the most recent end
      if (miss) sh.miss[misses + lru_mbcnt(mm)] = sh.dexp[d];
      hits += __popcll(hm);
      misses += __popcll(mm);
    }
    if (lane == 0) {
      sh.hits = hits;
      sh.misses = misses;
      sh.valid = valid;
    }
  }
  __syncthreads();
  const uint32_t H = sh.hits, M = sh.misses;

  // 2. every wave: the M smallest stamps of its slots (the hits now hold the
  //    newest stamps, and S >= N >= hits + M leaves M older slots)
  if (M > 0) {
    uint64_t st[kLruSlotsPerThread];
#pragma unroll
    for (int i = 0; i < kLruSlotsPerThread; ++i) {
      const uint32_t s = tid + static_cast<uint32_t>(i) * kLruThreads;
      st[i] = s < S ? p.slot_stamp[s] : kLruNoStamp;
    }
    uint32_t slot;
    uint64_t cur = lru_next(st, tid, S, 0, slot);
    uint32_t n = 0;
    for (; n < M; ++n) {
      const uint64_t v = wave_min_u64(cur);
      if (v == kLruNoStamp) break;
      const uint32_t owner = static_cast<uint32_t>(__builtin_ctzll(__ballot(cur == v)));
      const uint32_t vslot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(slot), owner));
      if (lane == 0) {
        sh.cand[wave][n] = v;
        sh.cslot[wave][n] = vslot;
      }
      if (lane == owner) cur = lru_next(st, tid, S, v, slot);
    }
    if (lane == 0) sh.ccount[wave] = n;
  }
  __syncthreads();

  // 3. one wave: merge, evict, map, stamp, list the fills, count
  if (wave == 0) {
    uint32_t found = 0;
    if (M > 0) {
      uint32_t head = 0;
      const uint32_t count = lane < kLruWaves ? sh.ccount[lane] : 0;
      uint64_t key = head < count ? sh.cand[lane][head] : kLruNoStamp;
      for (; found < M; ++found) {
        const uint64_t v = wave_min_u64(key);
        if (v == kLruNoStamp) break;  // only with a corrupted state: fewer slots than misses
        const uint32_t owner = static_cast<uint32_t>(__builtin_ctzll(__ballot(key == v)));
        if (lane == owner) {
          sh.victim[found] = sh.cslot[lane][head];
          ++head;
          key = head < count ? sh.cand[lane][head] : kLruNoStamp;
        }
      }
      if (found < M && lane == 0 && p.status != nullptr) atomicOr(p.status, 16u);
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      for (uint32_t m = lane; m < found; m += 64) {
        const uint32_t v = sh.victim[m];
        const int32_t e = sh.miss[m];
        const int32_t old = p.slot_owner[v];
        if (old >= 0 && static_cast<uint32_t>(old) < keys) p.slot_table[old] = -1;
        p.slot_owner[v] = static_cast<int32_t>(p.layer * E + static_cast<uint32_t>(e));
        table[e] = static_cast<int32_t>(v);
        p.slot_stamp[v] = base + 1 + H + m;
        const int32_t row = p.host_row[static_cast<size_t>(p.layer) * E + e];
        const bool ok = row >= 0 && static_cast<uint64_t>(row) < p.host_records;
        if (!ok && p.status != nullptr) atomicOr(p.status, 4u);
        p.fill_src[m] = ok ? static_cast<uint32_t>(row) : kNoRecord;
        p.fill_dst[m] = v;
      }
    }
    if (lane == 0) {
      uint64_t* layer_counters = p.counters + 4 + 4 * static_cast<size_t>(p.layer);
      const uint32_t valid = sh.valid;
      p.counters[0] = base + H + M;
      p.counters[1] += H;
      p.counters[2] += M;
      p.counters[3] += valid - M;
      layer_counters[0] += H;
      layer_counters[1] += M;
      layer_counters[2] += valid - M;
      layer_counters[3] += valid;
      *p.fill_count = found;
    }
  }
}

}  // namespace vm
