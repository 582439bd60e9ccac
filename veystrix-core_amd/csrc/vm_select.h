// Decode-path device helpers shared by the decode kernels and the fused
// experts kernel: register-resident activation groups, the router softmax and
// the top-k selection (gate desc, index asc) without a sort, route words.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kMaxExpertsPerLane = 8;  // expert_count <= 512

template <class A>
constexpr bool is_bf16() {
  return std::is_same<A, ActBF16>::value;
}

// One 32-input activation group in registers.  fetch() issues the loads,
// prepare() turns the raw values into the operands of the group dot.
template <class A>
struct GroupAct;

template <>
struct GroupAct<ActBF16> {
  uint32_t xp[16];  // after prepare(): pairs (x_{8i+n}, x_{8i+n+4}) at 4i+n
  float sum, sum128;
  __device__ __forceinline__ void fetch(const void* src, size_t elem) {
    const uint4* v = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + elem);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 r = v[q];
      xp[4 * q] = r.x; xp[4 * q + 1] = r.y; xp[4 * q + 2] = r.z; xp[4 * q + 3] = r.w;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 16; ++i) xp[i] = 0;
  }
  __device__ __forceinline__ void prepare() {
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) raw[i] = xp[i];
    pair_activations(raw, xp);
    sum = bf16_pair_sum(raw);
    sum128 = 128.0f * sum;
  }
  // scale * sum(q x) + bias * sum(x); the dot carries +128*sum(x)
  __device__ __forceinline__ float apply(const uint4 w, float s, float b) const {
    return fmaf(s, q4_dot_bf16(w, xp) - sum128, b * sum);
  }
};

template <>
struct GroupAct<ActF32> {
  float x[32];
  float sum;
  __device__ __forceinline__ void fetch(const void* src, size_t elem) {
    const float4* v = reinterpret_cast<const float4*>(static_cast<const float*>(src) + elem);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 r = v[q];
      x[4 * q] = r.x; x[4 * q + 1] = r.y; x[4 * q + 2] = r.z; x[4 * q + 3] = r.w;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] = 0.0f;
  }
  __device__ __forceinline__ void prepare() {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) s += x[4 * q] + x[4 * q + 1] + x[4 * q + 2] + x[4 * q + 3];
    sum = s;
  }
  __device__ __forceinline__ float apply(const uint4 w, float s, float b) const {
    return fmaf(s, q4_dot_f32(w, x), b * sum);
  }
};

__device__ __forceinline__ void flag(uint32_t* status, uint32_t bits) {
  if (status != nullptr) atomicOr(status, bits);
}

__device__ __forceinline__ uint32_t mbcnt(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// 1 KiB of zeros.  Lanes without data (tile tails, groups beyond the width,
// unresolved routes, empty slots) load from here instead of skipping the
// load: with the same number of loads on every path the compiler can wait for
// one early load without waiting for all later ones, and no load waits inside
// a branch.
__device__ uint4 g_zero_page[64];

// ------------------------------------------------------------- select -----
// Router softmax in fp32 over the E logits of one token, gates rounded to the
// activation type, then the top-K by (gate desc, index asc) and the
// renormalised scores.  One wave; lane l holds experts l + 64 m (m < 8).
//
// Selection without a sort: gates are >= 0, so their bit patterns order like
// their values.  A ballot binary search over the 64 lane maxima bounds the
// K-th largest gate from below; the few gates at or above the bound are
// compacted into LDS and ranked by comparing keys.  A block that runs one
// routed pair keeps only its own rank; the block that publishes the
// selection keeps all K.

// exp(x) for x <= 0 as 2^(x*log2 e) on v_exp_f32, with the rounding error of
// the product carried as a first-order correction (about 2 ulp in fp32).
__device__ __forceinline__ float exp_neg(float x) {
  constexpr float kLog2e = 1.44269502162933349609375f;  // log2(e) rounded to fp32
  constexpr float kLog2eLo = 1.925963033500011e-8f;     // log2(e) - kLog2e
  constexpr float kLn2 = 0.693147180559945309f;
  const float th = x * kLog2e;
  const float tl = fmaf(x, kLog2e, -th) + x * kLog2eLo;
  return __builtin_amdgcn_exp2f(th) * fmaf(tl, kLn2, 1.0f);
}

// Gate keys of one token: the gate's bit pattern (bf16: its upper 16 bits),
// 0 for lanes beyond E.  Lower expert indices win ties, so padding lanes
// (indices >= E) are never taken while K <= E.
template <class A>
struct GateKeys {
  static constexpr int kShift = is_bf16<A>() ? 16 : 0;
  static constexpr uint32_t kTop = 0x3f800000u >> kShift;  // key of gate 1.0
  uint32_t k[kMaxExpertsPerLane];
  __device__ static float gate(uint32_t key) { return __uint_as_float(key << kShift); }
};

// Lane l reads logits l + 64 m (clamped to E - 1, so every load is
// unconditional); entries beyond E become -FLT_MAX.
__device__ __forceinline__ void load_logits(const float* logits, uint32_t E, uint32_t lane,
                                            float l[kMaxExpertsPerLane]) {
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64u * m;
    const float v = logits[min(e, E - 1)];
    l[m] = e < E ? v : -FLT_MAX;
  }
}

template <class A>
__device__ void softmax_keys(const float l[kMaxExpertsPerLane], uint32_t E, uint32_t lane, GateKeys<A>& g) {
  float lmax = l[0];
#pragma unroll
  for (int m = 1; m < kMaxExpertsPerLane; ++m) lmax = fmaxf(lmax, l[m]);
  lmax = wave_max_f32(lmax);
  float ex[kMaxExpertsPerLane];
  float local = 0.0f;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    ex[m] = lane + 64u * m < E ? exp_neg(l[m] - lmax) : 0.0f;
    local += ex[m];
  }
  const float inv_total = 1.0f / wave_sum_all(local);
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64u * m;
    g.k[m] = e < E ? __float_as_uint(A::round(ex[m] * inv_total)) >> GateKeys<A>::kShift : 0u;
  }
}

// Number of keys >= v (wave-uniform).
template <class A>
__device__ __forceinline__ uint32_t count_ge(const GateKeys<A>& g, uint32_t v) {
  uint32_t c = 0;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) c += __popcll(__ballot(g.k[m] >= v));
  return c;
}

// Key of rank r: the largest v with more than r keys >= v.  `above` returns
// the number of keys > v (at most r).
template <class A>
__device__ uint32_t rank_key(const GateKeys<A>& g, uint32_t r, uint32_t& above) {
  uint32_t lo = 0, hi = GateKeys<A>::kTop + 1, c_hi = 0;  // count(>= lo) > r >= count(>= hi)
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    const uint32_t c = count_ge(g, mid);
    if (c > r) {
      lo = mid;
    } else {
      hi = mid;
      c_hi = c;
    }
  }
  above = c_hi;
  return lo;
}

// Candidates of the top K.  The K largest lane maxima are K distinct gates,
// so the K-th largest gate is at least the K-th largest lane maximum: every
// gate >= that bound is a candidate.  When more than kMaxCand gates reach the
// bound (many ties), the candidates are exactly the top K instead: the gates
// above the K-th largest key plus the lowest-index ties at it.  A candidate is
// stored as one key that orders like (gate desc, index asc): for bf16 gates
// (key << 9 | (511 - expert)) in 32 bits, for fp32 gates (key << 32 | ~expert)
// in 64 bits.  Returns their number (K..kMaxCand).
constexpr uint32_t kMaxCand = 64;

template <class A>
struct Cand {
  using T = typename std::conditional<is_bf16<A>(), uint32_t, uint64_t>::type;
  __device__ static T make(uint32_t key, uint32_t expert) {
    if constexpr (is_bf16<A>()) return (key << 9) | (511u - expert);
    else return (static_cast<uint64_t>(key) << 32) | (0xffffffffu - expert);
  }
  __device__ static uint32_t expert(T c) {
    if constexpr (is_bf16<A>()) return 511u - (c & 511u);
    else return 0xffffffffu - static_cast<uint32_t>(c);
  }
  __device__ static uint32_t key(T c) {
    if constexpr (is_bf16<A>()) return c >> 9;
    else return static_cast<uint32_t>(c >> 32);
  }
};

// First pass: every gate >= bound, in (m, lane) order.
template <class A>
__device__ __forceinline__ uint32_t compact_ge(const GateKeys<A>& g, uint32_t bound, uint32_t lane,
                                               typename Cand<A>::T* cand) {
  uint32_t c = 0;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const bool take = g.k[m] >= bound;
    const uint64_t sel = __ballot(take);
    const uint32_t pos = c + mbcnt(sel);
    if (take && pos < kMaxCand) cand[pos] = Cand<A>::make(g.k[m], lane + 64u * m);
    c += __popcll(sel);
  }
  return c;
}

// Exact top K when ties crowd the bound: the keys above `bound` and the
// first `need` ties at it in index order.
template <class A>
__device__ uint32_t compact_top(const GateKeys<A>& g, uint32_t bound, uint32_t need, uint32_t lane,
                                typename Cand<A>::T* cand) {
  uint32_t eq_before = 0, c = 0;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t k = g.k[m];
    const uint64_t eq = __ballot(k == bound);
    const bool take = k > bound || (k == bound && eq_before + mbcnt(eq) < need);
    const uint64_t sel = __ballot(take);
    const uint32_t pos = c + mbcnt(sel);
    if (take && pos < kMaxCand) cand[pos] = Cand<A>::make(k, lane + 64u * m);
    eq_before += __popcll(eq);
    c += __popcll(sel);
  }
  return c;
}

// K-th largest lane maximum: a search over the key range that tests three
// thresholds per step (independent ballots), two bits per step.
template <class A>
__device__ __forceinline__ uint32_t kth_lane_max(uint32_t lmax, uint32_t K) {
  uint32_t lo = 0, hi = GateKeys<A>::kTop + 1;  // count(lmax >= lo) >= K > count(lmax >= hi)
  while (hi - lo > 1) {
    const uint32_t q = (hi - lo + 3) >> 2;
    const uint32_t m1 = lo + q, m2 = min(lo + 2 * q, hi), m3 = min(lo + 3 * q, hi);
    const uint32_t c1 = __popcll(__ballot(lmax >= m1));
    const uint32_t c2 = __popcll(__ballot(lmax >= m2));
    const uint32_t c3 = __popcll(__ballot(lmax >= m3));
    if (c3 >= K) {
      lo = m3;
    } else if (c2 >= K) {
      lo = m2;
      hi = m3;
    } else if (c1 >= K) {
      lo = m1;
      hi = m2;
    } else {
      hi = m1;
    }
  }
  return lo;
}

template <class A>
__device__ uint32_t gather_candidates(const GateKeys<A>& g, uint32_t K, uint32_t lane, typename Cand<A>::T* cand) {
  uint32_t lmax = g.k[0];
#pragma unroll
  for (int m = 1; m < kMaxExpertsPerLane; ++m) lmax = max(lmax, g.k[m]);
  uint32_t c = compact_ge(g, kth_lane_max<A>(lmax, K), lane, cand);
  if (c > kMaxCand) {
    uint32_t above;
    const uint32_t vk = rank_key(g, K - 1, above);
    c = compact_top(g, vk, K - above, lane, cand);
  }
  __builtin_amdgcn_wave_barrier();
  return c;
}

// Rank of candidate `lane` among the c candidates (0 = largest gate); lanes
// >= c get `mine` = 0.
template <class A>
__device__ __forceinline__ uint32_t candidate_rank(const typename Cand<A>::T* cand, uint32_t c, uint32_t lane,
                                                   typename Cand<A>::T& mine) {
  mine = lane < c ? cand[lane] : 0u;
  uint32_t r = 0;
#pragma unroll 4
  for (uint32_t i = 0; i < c; ++i) r += cand[i] > mine ? 1u : 0u;
  return r;
}

// Expert of rank r < K (wave-uniform).
// bf16 gates: the top K by repeated wave maxima.  Every lane sorts its eight
// keys (gate << 9 | (511 - expert), unique, ordering like gate desc, index
// asc) with a 19-comparator network; then K rounds take the wave maximum of
// the lanes' heads (DPP) and the lane that owned it pops its head.  Only VALU
// and DPP work, no branch and no LDS: about 60% of the latency of the
// candidate search for K = 10 of 512.  Lane k < K returns the key of rank k;
// cand[0..K) receives the keys in rank order (for score_of_order).
__device__ __forceinline__ void sort8_desc(uint32_t k[8]) {
#define VM_CX(a, b)                  \
  {                                  \
    const uint32_t hi = max(k[a], k[b]); \
    const uint32_t lo = min(k[a], k[b]); \
    k[a] = hi;                       \
    k[b] = lo;                       \
  }
  VM_CX(0, 1) VM_CX(2, 3) VM_CX(4, 5) VM_CX(6, 7)
  VM_CX(0, 2) VM_CX(1, 3) VM_CX(4, 6) VM_CX(5, 7)
  VM_CX(1, 2) VM_CX(5, 6) VM_CX(0, 4) VM_CX(3, 7)
  VM_CX(1, 5) VM_CX(2, 6)
  VM_CX(1, 4) VM_CX(3, 6)
  VM_CX(2, 4) VM_CX(3, 5)
  VM_CX(3, 4)
#undef VM_CX
}

__device__ __forceinline__ uint32_t extract_top_bf16(const GateKeys<ActBF16>& g, uint32_t K, uint32_t lane,
                                                     uint32_t* cand) {
  uint32_t k[kMaxExpertsPerLane];
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) k[m] = (g.k[m] << 9) | (511u - (lane + 64u * m));
  sort8_desc(k);
  uint32_t mine = 0;
  for (uint32_t r = 0; r < K; ++r) {
    const uint32_t top = wave_max_u32(k[0]);
    if (lane == r) mine = top;
    const bool pop = k[0] == top;
#pragma unroll
    for (int m = 0; m < kMaxExpertsPerLane - 1; ++m) k[m] = pop ? k[m + 1] : k[m];
    k[kMaxExpertsPerLane - 1] = pop ? 0u : k[kMaxExpertsPerLane - 1];
  }
  if (lane < K) cand[lane] = mine;
  __builtin_amdgcn_wave_barrier();
  return mine;
}

template <class A>
__device__ typename Cand<A>::T rank_order(const GateKeys<A>& g, uint32_t K, uint32_t lane,
                                          typename Cand<A>::T* cand);

template <class A>
__device__ uint32_t select_rank(const GateKeys<A>& g, uint32_t K, uint32_t r, uint32_t lane,
                                typename Cand<A>::T* cand) {
  if constexpr (is_bf16<A>()) {
    // ranks 0..r are the first r + 1 wave maxima
    const uint32_t key = extract_top_bf16(g, r + 1, lane, cand);
    return Cand<A>::expert(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), r)));
  }
  const uint32_t c = gather_candidates(g, K, lane, cand);
  typename Cand<A>::T mine;
  const uint32_t rank = candidate_rank<A>(cand, c, lane, mine);
  const uint64_t hit = __ballot(lane < c && rank == r);
  const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(hit));
  if constexpr (is_bf16<A>()) {
    return Cand<A>::expert(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mine), src)));
  } else {
    return Cand<A>::expert(readlane_u64(mine, src));
  }
}

// The whole selection in rank order: lane k < K returns the expert of rank k
// and its renormalised score.  scores = gate / (mass + blend*(selected_mass
// - mass)), each step rounded to the activation type; the mass is summed in
// rank order.
// The top K in rank order: lane k < K returns the candidate of rank k (0 for
// the other lanes), and cand[0..K) holds them in that order afterwards.
template <class A>
__device__ typename Cand<A>::T rank_order(const GateKeys<A>& g, uint32_t K, uint32_t lane,
                                          typename Cand<A>::T* cand) {
  if constexpr (is_bf16<A>()) {
    return extract_top_bf16(g, K, lane, cand);
  } else {
    const uint32_t c = gather_candidates(g, K, lane, cand);
    typename Cand<A>::T mine;
    const uint32_t rank = candidate_rank<A>(cand, c, lane, mine);
    __builtin_amdgcn_wave_barrier();
    if (lane < c && rank < K) cand[rank] = mine;
    __builtin_amdgcn_wave_barrier();
    return lane < K ? cand[lane] : 0u;
  }
}

// Renormalised score of lane k's candidate `top` (rank order in cand[0..K)):
// gate / (mass + blend*(selected_mass - mass)), each step rounded to the
// activation type, blend included (the reference multiplies by blend as a
// scalar of the scores' type); the mass is summed in rank order.
template <class A>
__device__ float score_of_order(const typename Cand<A>::T* cand, typename Cand<A>::T top, uint32_t K, float blend,
                                uint32_t lane) {
  float mass = 0.0f;
  for (uint32_t i = 0; i < K; ++i) mass += GateKeys<A>::gate(Cand<A>::key(cand[i]));
  mass = A::round(mass);
  const float diff = A::round(mass - mass);
  const float normalizer = A::round(mass + A::round(A::round(blend) * diff));
  return lane < K ? A::round(GateKeys<A>::gate(Cand<A>::key(top)) / normalizer) : 0.0f;
}

template <class A>
__device__ void rank_selection(const GateKeys<A>& g, uint32_t K, float blend, uint32_t lane,
                               typename Cand<A>::T* cand, uint32_t& e_out, float& score_out) {
  const typename Cand<A>::T top = rank_order<A>(g, K, lane, cand);
  e_out = lane < K ? Cand<A>::expert(top) : 0u;
  score_out = score_of_order<A>(cand, top, K, blend, lane);
}

// dot of 8 bf16 weights with 8 activations (one 16-byte chunk)
template <class A>
struct RouterChunk;

template <>
struct RouterChunk<ActBF16> {
  uint4 x;
  __device__ __forceinline__ void load(const void* base, size_t elem) {
    x = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
  }
  __device__ __forceinline__ void zero() { x = make_uint4(0, 0, 0, 0); }
  __device__ __forceinline__ float dot(const uint4 w, float acc) const {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x), __builtin_bit_cast(bf16x2, x.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y), __builtin_bit_cast(bf16x2, x.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z), __builtin_bit_cast(bf16x2, x.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w), __builtin_bit_cast(bf16x2, x.w), acc, false);
    return acc;
  }
};

template <>
struct RouterChunk<ActF32> {
  float4 a, b;
  __device__ __forceinline__ void load(const void* base, size_t elem) {
    const float4* v = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    a = v[0];
    b = v[1];
  }
  __device__ __forceinline__ void zero() { a = b = make_float4(0, 0, 0, 0); }
  __device__ __forceinline__ float dot(const uint4 w, float acc) const {
    acc = fmaf(bf16_to_f32(w.x & 0xffffu), a.x, acc);
    acc = fmaf(bf16_to_f32(w.x >> 16), a.y, acc);
    acc = fmaf(bf16_to_f32(w.y & 0xffffu), a.z, acc);
    acc = fmaf(bf16_to_f32(w.y >> 16), a.w, acc);
    acc = fmaf(bf16_to_f32(w.z & 0xffffu), b.x, acc);
    acc = fmaf(bf16_to_f32(w.z >> 16), b.y, acc);
    acc = fmaf(bf16_to_f32(w.w & 0xffffu), b.z, acc);
    acc = fmaf(bf16_to_f32(w.w >> 16), b.w, acc);
    return acc;
  }
};

// Tokens per row of router blocks (grid y), and tokens whose activations a
// router wave loads together before their dot products.
constexpr uint32_t kFrontTokens = 8;
#ifndef VM_FRONT_UNROLL
#define VM_FRONT_UNROLL 4
#endif
constexpr int kFrontUnroll = VM_FRONT_UNROLL;

// One router row per wave over tokens [t_begin, t_end).  CH = 16-byte chunks
// per lane per row (hidden/512, rounded up).  U tokens at a time: their loads
// are issued together (tokens past the end repeat the last one and are not
// stored), so a row costs one load latency per U tokens.
template <class A, int CH, int U>
__device__ void router_row(const FrontLaunch& p, uint32_t row, uint32_t lane, uint32_t t_begin, uint32_t t_end) {
  const uint32_t H = p.hidden;
  uint4 w[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint32_t e8 = 8 * (lane + 64 * c);
    w[c] = e8 < H ? *reinterpret_cast<const uint4*>(p.weight + static_cast<size_t>(row) * H + e8)
                  : make_uint4(0, 0, 0, 0);
  }
  for (uint32_t t0 = t_begin; t0 < t_end; t0 += U) {
    float acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t t = min(t0 + u, t_end - 1);
      acc[u] = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t e8 = 8 * (lane + 64 * c);
        RouterChunk<A> xc;
        if (e8 < H) xc.load(p.x, static_cast<size_t>(t) * H + e8); else xc.zero();
        acc[u] = xc.dot(w[c], acc[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = group_sum<64>(acc[u]);
    if (lane == 63) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u >= t_end) break;
        float v = acc[u];
        if (p.bias != nullptr) v += p.bias[row];
        p.logits[static_cast<size_t>(t0 + u) * p.experts + row] = A::round(v);
      }
    }
  }
}

// The shared expert's H -> 1 quantized gate followed by the sigmoid, for one token.
template <class A>
__device__ void shared_gate_token(const FrontLaunch& p, uint32_t t, uint32_t lane) {
  const uint32_t H = p.hidden, G = H / kGroup;
  float acc = 0.0f;
  for (uint32_t g = lane; g < G; g += 64) {
    const uint4 w = *reinterpret_cast<const uint4*>(p.seg.w + g * kWordsPerGroup);
    GroupAct<A> xa;
    xa.fetch(p.x, static_cast<size_t>(t) * H + g * kGroup);
    xa.prepare();
    acc += xa.apply(w, bf16_to_f32(p.seg.s[g]), bf16_to_f32(p.seg.b[g]));
  }
  const float logit = A::round(wave_sum_all(acc));
  if (lane == 0) A::store(p.shared_sig, t, sigmoid_act<A>(logit));
}

__device__ __forceinline__ uint32_t route_word(int32_t slot) {
  return slot >= 0 ? (kSlotBit | static_cast<uint32_t>(slot)) : kMissWord;
}

}  // namespace

}  // namespace vm
