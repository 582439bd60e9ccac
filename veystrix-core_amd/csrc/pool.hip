// Device-resident LRU of the expert pool and the miss fill from pinned host
// memory (gfx950).
//
//   k_lru_assign  one block applies the reference's ExpertPool.assign
//                 (models/flashnext/expert_pool.py:123-159) to the routed ids
//                 of one decode call.  Recency is a per-slot stamp (all
//                 distinct; free slots carry the smallest, in pop order): the
//                 hits of the call get the next stamps in first-seen order,
//                 then the misses take the slots with the smallest remaining
//                 stamps, oldest first, and get the stamps after those.  That
//                 is the OrderedDict's move_to_end / popitem(last=False) order.
//                 The victims are found without a sort: every wave extracts the
//                 M smallest stamps of its slots (M = misses of the call), and
//                 one wave merges the 16 sorted lists.
//   k_pool_fill   the missed records, read by the GPU straight from pinned
//                 host memory (the reads run at the rate of a DMA copy) and
//                 written into their slots: no host round trip, no copy
//                 engine, nothing for the host to wait for.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kLruThreads = 1024;
constexpr int kLruWaves = kLruThreads / 64;
constexpr int kFillThreads = 256;
constexpr int kFillBlocks = 128;  // 128 blocks of 4 loads in flight per thread saturate the host link
constexpr uint64_t kNoStamp = ~0ull;

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ uint32_t lane_mbcnt(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Smallest stamp above `floor` among the slots of this thread (kNoStamp if none).
__device__ __forceinline__ uint64_t next_stamp(const uint64_t* stamp, uint32_t slots, uint32_t first, uint64_t floor,
                                               uint32_t& slot) {
  uint64_t best = kNoStamp;
  slot = 0;
  for (uint32_t s = first; s < slots; s += kLruThreads) {
    const uint64_t v = stamp[s];
    if (v > floor && v < best) {
      best = v;
      slot = s;
    }
  }
  return best;
}

__global__ __launch_bounds__(kLruThreads) void k_lru_assign(LruLaunch p) {
  __shared__ int32_t s_routed[kLruMaxRouted];  // routed ids, -1 when out of range
  __shared__ int32_t s_dexp[kLruMaxRouted];    // distinct ids in first-seen order
  __shared__ int32_t s_dslot[kLruMaxRouted];   // their slots, -1 on a miss
  __shared__ int32_t s_miss[kLruMaxRouted];    // missed ids in first-seen order
  __shared__ uint64_t s_cand[kLruWaves][kLruMaxRouted];
  __shared__ uint32_t s_cslot[kLruWaves][kLruMaxRouted];
  __shared__ uint32_t s_ccount[kLruWaves];
  __shared__ uint32_t s_victim[kLruMaxRouted];
  __shared__ uint32_t s_hits, s_misses, s_valid;
  __shared__ uint64_t s_base;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t N = p.routed;
  const uint32_t E = p.experts;
  const uint32_t S = p.slots;
  const uint32_t keys = p.layers * E;
  int32_t* table = p.slot_table + static_cast<size_t>(p.layer) * E;

  // 1. the routed ids and the last stamp issued
  if (tid < N) {
    const int32_t e = p.inds[tid];
    const bool ok = e >= 0 && static_cast<uint32_t>(e) < E;
    s_routed[tid] = ok ? e : -1;
    if (!ok && p.status != nullptr) atomicOr(p.status, 8u);
  }
  if (tid == 0) s_base = p.counters[0];
  __syncthreads();
  const uint64_t base = s_base;

  // 2. one wave: distinct ids in first-seen order, their slots, hits and misses
  if (wave == 0) {
    uint32_t nd = 0, valid = 0;
    for (uint32_t c = 0; c < N; c += 64) {
      const uint32_t i = c + lane;
      const int32_t e = i < N ? s_routed[i] : -1;
      bool first = e >= 0;
      for (uint32_t j = 0; j < i && first; ++j) first = s_routed[j] != e;
      valid += __popcll(__ballot(e >= 0));
      const uint64_t fm = __ballot(first);
      if (first) {
        const uint32_t d = nd + lane_mbcnt(fm);
        const int32_t slot = table[e];
        s_dexp[d] = e;
        s_dslot[d] = slot >= 0 && static_cast<uint32_t>(slot) < S ? slot : -1;
      }
      nd += __popcll(fm);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    uint32_t hits = 0, misses = 0;
    for (uint32_t c = 0; c < nd; c += 64) {
      const uint32_t d = c + lane;
      const int32_t slot = d < nd ? s_dslot[d] : -1;
      const bool hit = d < nd && slot >= 0;
      const bool miss = d < nd && slot < 0;
      const uint64_t hm = __ballot(hit), mm = __ballot(miss);
      // hits move to the most recent end in first-seen order
      if (hit) p.slot_stamp[slot] = base + 1 + hits + lane_mbcnt(hm);
      if (miss) s_miss[misses + lane_mbcnt(mm)] = s_dexp[d];
      hits += __popcll(hm);
      misses += __popcll(mm);
    }
    if (lane == 0) {
      s_hits = hits;
      s_misses = misses;
      s_valid = valid;
    }
  }
  __syncthreads();
  const uint32_t H = s_hits, M = s_misses;

  // 3. every wave: the M smallest stamps of its slots (hit slots now hold the
  //    newest stamps; S >= N >= hits + M leaves M older slots)
  if (M > 0) {
    uint32_t slot;
    uint64_t cur = next_stamp(p.slot_stamp, S, tid, 0, slot);
    uint32_t n = 0;
    for (; n < M; ++n) {
      const uint64_t v = wave_min_u64(cur);
      if (v == kNoStamp) break;
      const uint32_t owner = static_cast<uint32_t>(__builtin_ctzll(__ballot(cur == v)));
      const uint32_t vslot = __builtin_amdgcn_readlane(slot, owner);
      if (lane == 0) {
        s_cand[wave][n] = v;
        s_cslot[wave][n] = vslot;
      }
      if (lane == owner) cur = next_stamp(p.slot_stamp, S, tid, v, slot);
    }
    if (lane == 0) s_ccount[wave] = n;
  }
  __syncthreads();

  // 4. one wave: merge the per-wave lists, evict, map, stamp, list the fills
  if (wave == 0) {
    uint32_t found = 0;
    if (M > 0) {
      uint32_t head = 0;
      const uint32_t count = lane < kLruWaves ? s_ccount[lane] : 0;
      uint64_t key = head < count ? s_cand[lane][head] : kNoStamp;
      for (; found < M; ++found) {
        const uint64_t v = wave_min_u64(key);
        if (v == kNoStamp) break;  // only with a corrupted state: fewer slots than misses
        const uint32_t owner = static_cast<uint32_t>(__builtin_ctzll(__ballot(key == v)));
        if (lane == owner) {
          s_victim[found] = s_cslot[lane][head];
          ++head;
          key = head < count ? s_cand[lane][head] : kNoStamp;
        }
      }
      if (found < M && lane == 0 && p.status != nullptr) atomicOr(p.status, 16u);
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      for (uint32_t m = lane; m < found; m += 64) {
        const uint32_t v = s_victim[m];
        const int32_t e = s_miss[m];
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
      p.counters[0] = base + H + M;
      p.counters[1] += H;
      p.counters[2] += M;
      p.counters[3] += s_valid - M;
      layer_counters[0] += H;
      layer_counters[1] += M;
      layer_counters[2] += s_valid - M;
      layer_counters[3] += s_valid;
      *p.fill_count = found;
    }
  }
}

__global__ __launch_bounds__(kFillThreads) void k_pool_fill(FillLaunch p) {
  const uint32_t M = min(*p.count, kLruMaxRouted);
  const uint64_t units = p.record_bytes / 16;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kFillThreads;
  for (uint32_t m = 0; m < M; ++m) {
    const uint32_t src = p.src[m], dst = p.dst[m];
    if (src >= p.host_records || dst >= p.pool_records) continue;
    const uint4* s = reinterpret_cast<const uint4*>(p.host + static_cast<uint64_t>(src) * p.host_stride);
    uint4* d = reinterpret_cast<uint4*>(p.pool + p.header + static_cast<uint64_t>(dst) * p.stride);
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * kFillThreads + threadIdx.x;
    for (; i + 3 * stride < units; i += 4 * stride) {
      const uint4 a = s[i], b = s[i + stride], c = s[i + 2 * stride], e = s[i + 3 * stride];
      d[i] = a;
      d[i + stride] = b;
      d[i + 2 * stride] = c;
      d[i + 3 * stride] = e;
    }
    for (; i < units; i += stride) d[i] = s[i];
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

}  // namespace

hipError_t launch_lru(const LruLaunch& p, hipStream_t stream) {
  return launch("lru", k_lru_assign, dim3(1), dim3(kLruThreads), stream, p);
}

hipError_t launch_fill(const FillLaunch& p, hipStream_t stream) {
  return launch("fill", k_pool_fill, dim3(kFillBlocks), dim3(kFillThreads), stream, p);
}

}  // namespace vm
