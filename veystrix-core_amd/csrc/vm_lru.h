// Device side of the expert pool's LRU (one block of kLruThreads threads).
//
// The reference's ExpertPool.assign (models/flashnext/expert_pool.py:123-159)
// on one queue of slot ids, least recently used first: the free slots in the
// order the reference's free list pops them, then the OrderedDict's resident
// slots.  A call moves its hits to the most recent end in first-seen order,
// then each miss takes the next victim, which is the first queue entry that
// is not a hit (free slots first, then the oldest key) and goes to the end.
// So the queue after the call is
//
//     [non-hit entries after the first M] [hits, first-seen order] [victims, miss order]
//
// and the call is one order-preserving compaction of the queue: each thread
// holds a contiguous run of entries in registers, a block-wide prefix count of
// the non-hit entries gives every entry its new position, and the entries
// whose count is below M are the victims; thread m then evicts victim m and
// maps miss m to it.  No step is serial in the number of misses.
//
// Latency: the call is a chain of small dependent steps, so what does not
// depend on the routed ids (queue, owners, counters) is loaded while the
// selection runs, the slot and host row of every routed id are loaded
// together, and the block barriers wait on LDS only (global stores stay in
// flight).  Nothing global is written before the state has been checked.
#pragma once

#include "vm_internal.h"

namespace vm {

constexpr int kLruWaves = kLruThreads / 64;
constexpr uint32_t kLruMaxExperts = 512;   // ids index an LDS map of this size
constexpr int kLruChunks = (kLruMaxRouted + 63) / 64;

struct LruShared {
  uint32_t first[kLruMaxExperts];   // first position of each id in the routed list
  uint32_t hit_bits[kLruThreads];   // bit i of word w: slot w + kLruThreads * i is a hit
  int32_t miss[kLruMaxRouted];      // missed ids in first-seen order
  int32_t miss_row[kLruMaxRouted];  // their host rows
  int32_t hit_slot[kLruMaxRouted];  // slots of the hits in first-seen order
  int32_t victim[kLruMaxRouted];    // victim slots, oldest first
  int32_t vowner[kLruMaxRouted];    // their owner keys before the call
  uint32_t wsum[kLruWaves];         // per wave: non-hit entries | hit entries << 16
  uint32_t wbad[kLruWaves];         // per wave: entries outside 0..slots-1
  uint64_t counter[8];              // counters[0..3], then the layer's four, before the call
  uint32_t hits, misses, valid;
};

// Per-thread state loaded before the routed ids are known.  P bounds the
// queue entries a thread holds (at least ceil(order_len / kLruThreads)): the
// per-entry loops run P iterations, so the kernel is instantiated for the
// powers of two up to kLruSlotsPerThread and launched with the smallest that
// fits the queue.
template <int P>
struct LruRegs {
  int32_t q[P];                      // queue entries lo .. lo + n - 1
  int32_t own[P];                    // owners of those slots
  uint32_t lo, n;
  uint64_t counter;                  // wave 0, lanes 0..7: counters[0..3], then the layer's four
};

__device__ __forceinline__ uint32_t lru_mbcnt(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, uint32_t lane) {
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    const uint32_t u = static_cast<uint32_t>(__shfl_up(static_cast<int>(v), d, 64));
    if (lane >= d) v += u;
  }
  return v;
}

// Every thread, before the selection: clear the LDS maps, load this thread's
// run of the queue and (wave 0) the counters.  A block barrier must separate
// it from lru_assign.
template <int P>
__device__ __forceinline__ void lru_begin(const LruLaunch& p, LruShared& sh, LruRegs<P>& r) {
  const uint32_t tid = threadIdx.x;
  if (tid < kLruMaxExperts) sh.first[tid] = ~0u;
  sh.hit_bits[tid] = 0;
  const uint32_t U = p.order_len;
  const uint32_t per = (U + kLruThreads - 1) / kLruThreads;  // <= P
  r.lo = tid * per;
  r.n = r.lo < U ? min(per, U - r.lo) : 0u;
#pragma unroll
  for (int i = 0; i < P; ++i)
    r.q[i] = static_cast<uint32_t>(i) < r.n ? p.lru_order[r.lo + i] : -1;
  const uint32_t lane = tid & 63u;
  r.counter = 0;
  if (tid < 8) r.counter = p.counters[lane < 4 ? lane : 4 + 4 * static_cast<size_t>(p.layer) + (lane - 4)];
}

// Every thread, after the selection (its registers are free by then): the
// owners of this thread's queue entries, in flight while wave 0 looks up the
// routed ids.
template <int P>
__device__ __forceinline__ void lru_owners(const LruLaunch& p, LruRegs<P>& r) {
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int32_t s = r.q[i];
    r.own[i] = static_cast<uint32_t>(i) < r.n && s >= 0 && static_cast<uint32_t>(s) < p.slots ? p.slot_owner[s] : -1;
  }
}

// assign() of the routed ids in `routed` (LDS, -1 = skipped) for one call.
// Every thread of the block must call it (it holds block barriers).
template <int P>
__device__ void lru_assign(const LruLaunch& p, const int32_t* routed, LruShared& sh, LruRegs<P>& r) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t N = p.routed, E = p.experts, S = p.slots;
  const uint32_t keys = p.layers * E;
  int32_t* table = p.slot_table + static_cast<size_t>(p.layer) * E;
  const int32_t* rows = p.host_row + static_cast<size_t>(p.layer) * E;

  // 1. one wave: slots and host rows of every routed id (loads issued together),
  //    first occurrences through the LDS map, hits and misses listed in LDS
  if (wave == 0) {
    int32_t e[kLruChunks], slot[kLruChunks], row[kLruChunks];
    uint32_t valid = 0;
    bool bad = false;
#pragma unroll
    for (int c = 0; c < kLruChunks; ++c) {
      const uint32_t i = 64u * c + lane;
      int32_t id = i < N ? routed[i] : -1;
      if (id >= 0 && static_cast<uint32_t>(id) >= E) {
        bad = true;
        id = -1;
      }
      e[c] = id;
      slot[c] = -1;
      row[c] = -1;
      if (id >= 0) {
        atomicMin(&sh.first[id], i);
        slot[c] = table[id];
        row[c] = rows[id];
      }
      valid += __popcll(__ballot(id >= 0));
    }
    if (__ballot(bad) != 0 && lane == 0 && p.status != nullptr) atomicOr(p.status, 8u);
    if (lane < 8) sh.counter[lane] = r.counter;
    uint32_t hits = 0, misses = 0;
#pragma unroll
    for (int c = 0; c < kLruChunks; ++c) {
      const uint32_t i = 64u * c + lane;
      const bool first = e[c] >= 0 && sh.first[e[c]] == i;
      const bool hit = first && slot[c] >= 0 && static_cast<uint32_t>(slot[c]) < S;
      const bool miss = first && !hit;
      const uint64_t hm = __ballot(hit), mm = __ballot(miss);
      if (hit) {
        const uint32_t s = static_cast<uint32_t>(slot[c]);
        sh.hit_slot[hits + lru_mbcnt(hm)] = slot[c];
        atomicOr(&sh.hit_bits[s % kLruThreads], 1u << (s / kLruThreads));
      }
      if (miss) {
        const uint32_t m = misses + lru_mbcnt(mm);
        sh.miss[m] = e[c];
        sh.miss_row[m] = row[c];
      }
      hits += __popcll(hm);
      misses += __popcll(mm);
    }
    if (lane == 0) {
      sh.hits = hits;
      sh.misses = misses;
      sh.valid = valid;
    }
  }
  lds_barrier();
  const uint32_t H = sh.hits, M = sh.misses;

  // 2. every thread: classify its entries (kept = not a hit), prefix count of
  //    the kept entries within the wave, wave totals to LDS
  uint32_t keep_mask = 0, keep = 0, hitq = 0, bad = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (static_cast<uint32_t>(i) < r.n) {
      const int32_t s = r.q[i];
      if (s < 0 || static_cast<uint32_t>(s) >= S) {
        ++bad;
      } else if ((sh.hit_bits[s % kLruThreads] >> (s / kLruThreads)) & 1u) {
        ++hitq;
      } else {
        keep_mask |= 1u << i;
        ++keep;
      }
    }
  }
  const uint32_t packed = keep | (hitq << 16);  // wave and block totals stay below 2^16 in each half
  const uint32_t incl = wave_inclusive_sum(packed, lane);
  if (lane == 63) sh.wsum[wave] = incl;
  const bool wave_bad = __ballot(bad != 0) != 0;
  if (lane == 0) sh.wbad[wave] = wave_bad ? 1u : 0u;
  lds_barrier();

  uint32_t before = 0, total = 0, any_bad = 0;
#pragma unroll
  for (int w = 0; w < kLruWaves; ++w) {
    const uint32_t v = sh.wsum[w];
    before += static_cast<uint32_t>(w) < wave ? v : 0u;
    total += v;
    any_bad |= sh.wbad[w];
  }
  const uint32_t NH = total & 0xffffu, HQ = total >> 16;
  if (any_bad != 0 || HQ != H) {  // not a queue of this pool's hits: leave the state untouched
    if (tid == 0) {
      if (p.status != nullptr) atomicOr(p.status, 16u);
      *p.fill_count = 0;
    }
    return;
  }

  // 3. every thread: move its kept entries up, list its victims
  const uint32_t found = min(M, NH);
  const uint32_t kept = NH - found;
  uint32_t rank = (before + incl - packed) & 0xffffu;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if ((keep_mask >> i) & 1u) {
      if (rank < found) {
        sh.victim[rank] = r.q[i];
        sh.vowner[rank] = r.own[i];
      } else if (rank - found != r.lo + static_cast<uint32_t>(i)) {
        p.lru_order[rank - found] = r.q[i];
      }
      ++rank;
    }
  }
  if (tid < H) p.lru_order[kept + tid] = sh.hit_slot[tid];
  lds_barrier();

  // 4. thread m < found: evict victim m, map miss m to it, list its fill
  if (tid < found) {
    const uint32_t m = tid;
    const int32_t v = sh.victim[m];
    const int32_t old = sh.vowner[m];
    const int32_t e = sh.miss[m];
    const int32_t row = sh.miss_row[m];
    if (old >= 0 && static_cast<uint32_t>(old) < keys) p.slot_table[old] = -1;
    p.slot_owner[v] = static_cast<int32_t>(p.layer * E + static_cast<uint32_t>(e));
    table[e] = v;
    p.lru_order[kept + H + m] = v;
    const bool ok = row >= 0 && static_cast<uint64_t>(row) < p.host_records;
    if (!ok && p.status != nullptr) atomicOr(p.status, 4u);
    p.fill_src[m] = ok ? static_cast<uint32_t>(row) : kNoRecord;
    p.fill_dst[m] = static_cast<uint32_t>(v);
  }
  if (tid == 0) {
    *p.fill_count = found;
    if (found < M && p.status != nullptr) atomicOr(p.status, 16u);
  }
  // counters: lanes 0..3 pool-wide, lanes 4..7 the layer's hits, misses, routed hits, routed ids
  if (tid < 8) {
    const uint32_t valid = sh.valid;
    const uint64_t add[8] = {H + M, H, M, valid - M, H, M, valid - M, valid};
    uint64_t d = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) d = lane == static_cast<uint32_t>(k) ? add[k] : d;
    p.counters[lane < 4 ? lane : 4 + 4 * static_cast<size_t>(p.layer) + (lane - 4)] = sh.counter[lane] + d;
  }
}

}  // namespace vm
