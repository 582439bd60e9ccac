// Decode kernels of the routed-expert MoE layer for gfx950 (wave64).
//
// A decode layer is three launches with no in-kernel cross-block sync (a
// device-scope fence costs more than a kernel boundary on this part):
//
//   k_front   router logits x . Wr^T (one row per wave, bf16 dot2) and the
//             shared expert's H -> 1 Q4 gate with its sigmoid.
//   k_gateup  every block of a routed pair first recomputes softmax + top-k
//             of its token from the logits (identical in every block), maps
//             the selected expert to its pool slot through an LDS copy of
//             the slot table, then streams the gate and up Q4/G32 rows with
//             SwiGLU in a block-parallel epilogue.  Shared-expert pairs skip
//             the selection.  One block per token publishes indices, scores
//             and route words for k_down.
//   k_down    down Q4/G32 GEMV of every slot of a token for a tile of output
//             rows, then the router-score combine with the shared term.
//   k_select  softmax + top-k alone (router entry point, split layer path).
//
// Bandwidth layout: one 16-byte load per lane covers one 32-input group of a
// row (4 packed words); scale and bias are 2-byte loads that coalesce into one
// 128-byte line per row; activations are staged once per block in LDS,
// pre-paired for v_dot2 with the group sums alongside; row sums use DPP.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kMaxExpertsPerLane = 8;  // expert_count <= 512
constexpr int kMaxTopK = 16;

template <class A>
constexpr bool is_bf16() {
  return std::is_same<A, ActBF16>::value;
}

// LDS words per 32-input group: bf16 16 pair words + sum + 128*sum (+2 pad);
// f32 32 values + sum (+3 pad).  Strides of 20 / 36 words keep 16 lanes of
// consecutive groups on distinct banks for 16-byte reads.
template <class A>
constexpr int lds_group_words() {
  return is_bf16<A>() ? 20 : 36;
}

// Stage the 32 activations of group g (elements elem..elem+31) into LDS.
template <class A>
__device__ __forceinline__ void stage_group(const void* src, size_t elem, uint32_t* dst) {
  if constexpr (is_bf16<A>()) {
    const uint4* v = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + elem);
    uint32_t raw[16], xp[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 r = v[q];
      raw[4 * q + 0] = r.x; raw[4 * q + 1] = r.y; raw[4 * q + 2] = r.z; raw[4 * q + 3] = r.w;
    }
    pair_activations(raw, xp);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      reinterpret_cast<uint4*>(dst)[q] = make_uint4(xp[4 * q], xp[4 * q + 1], xp[4 * q + 2], xp[4 * q + 3]);
    const float s = bf16_pair_sum(raw);
    reinterpret_cast<uint2*>(dst)[8] = make_uint2(__float_as_uint(s), __float_as_uint(128.0f * s));
  } else {
    const float4* v = reinterpret_cast<const float4*>(static_cast<const float*>(src) + elem);
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 r = v[q];
      reinterpret_cast<float4*>(dst)[q] = r;
      s += r.x + r.y + r.z + r.w;
    }
    dst[32] = __float_as_uint(s);
  }
}

__device__ __forceinline__ void stage_zero(uint32_t* dst, int words) {
  for (int i = 0; i < words; ++i) dst[i] = 0;
}

// One group's activations in registers, read back from LDS.
template <class A>
struct GroupAct;

template <>
struct GroupAct<ActBF16> {
  uint32_t xp[16];
  float sum, sum128;
  __device__ __forceinline__ void load_lds(const uint32_t* src) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 r = reinterpret_cast<const uint4*>(src)[q];
      xp[4 * q] = r.x; xp[4 * q + 1] = r.y; xp[4 * q + 2] = r.z; xp[4 * q + 3] = r.w;
    }
    const uint2 s = reinterpret_cast<const uint2*>(src)[8];
    sum = __uint_as_float(s.x);
    sum128 = __uint_as_float(s.y);
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
  __device__ __forceinline__ void load_lds(const uint32_t* src) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 r = reinterpret_cast<const float4*>(src)[q];
      x[4 * q] = r.x; x[4 * q + 1] = r.y; x[4 * q + 2] = r.z; x[4 * q + 3] = r.w;
    }
    sum = __uint_as_float(src[32]);
  }
  __device__ __forceinline__ float apply(const uint4 w, float s, float b) const {
    return fmaf(s, q4_dot_f32(w, x), b * sum);
  }
};

__device__ __forceinline__ void flag(uint32_t* status, uint32_t bits) {
  if (status != nullptr) atomicOr(status, bits);
}

// ------------------------------------------------------------- select -----
// Softmax over the E logits of one token (fp32), gates rounded to the
// activation type, top-K by (gate desc, index asc), renormalised scores.
// One wave; lane k < K returns rank k.  Lanes hold experts lane + 64*m; each
// lane sorts its keys, then K rounds take the wave-wide max of the list heads.

template <class A>
struct SelectKey {
  using T = uint32_t;  // bf16: (gate bits << 16) | (0xffff - e); 0 = empty
  __device__ static T make(float gate, uint32_t e) { return (f32_to_bf16(gate) << 16) | (0xffffu - e); }
  __device__ static T wave_max(T v) { return wave_max_u32(v); }
  __device__ static uint32_t expert(T k) { return 0xffffu - (k & 0xffffu); }
  __device__ static float gate(T k) { return bf16_to_f32(k >> 16); }
};

template <>
struct SelectKey<ActF32> {
  using T = uint64_t;  // (gate bits << 32) | (0xffffffff - e)
  __device__ static T make(float gate, uint32_t e) {
    return (static_cast<uint64_t>(__float_as_uint(gate)) << 32) | (0xffffffffu - e);
  }
  __device__ static T wave_max(T v) {
    const uint32_t hi = wave_max_u32(static_cast<uint32_t>(v >> 32));
    const uint32_t lo = wave_max_u32(static_cast<uint32_t>(v >> 32) == hi ? static_cast<uint32_t>(v) : 0u);
    return (static_cast<uint64_t>(hi) << 32) | lo;
  }
  __device__ static uint32_t expert(T k) { return 0xffffffffu - static_cast<uint32_t>(k); }
  __device__ static float gate(T k) { return __uint_as_float(static_cast<uint32_t>(k >> 32)); }
};

template <class T>
__device__ __forceinline__ void cas_desc(T& a, T& b) {
  const T hi = a > b ? a : b;
  const T lo = a > b ? b : a;
  a = hi;
  b = lo;
}

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

// Orderable integer image of a float (monotone for all non-NaN values).
__device__ __forceinline__ int float_order(float f) {
  const int b = __float_as_int(f);
  return b >= 0 ? b : (b ^ 0x7fffffff);
}

__device__ __forceinline__ float order_float(int k) {
  return __int_as_float(k >= 0 ? k : (k ^ 0x7fffffff));
}

__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, static_cast<int>(dpp_u<kDppQuadXor1>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int>(dpp_u<kDppQuadXor2>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int>(dpp_u<kDppHalfMirror>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int>(dpp_u<kDppMirror>(static_cast<uint32_t>(v))));
  const int t15 = __builtin_amdgcn_update_dpp(v, v, kDppBcast15, 0xA, 0xF, false);
  v = max(v, t15);
  const int t31 = __builtin_amdgcn_update_dpp(v, v, kDppBcast31, 0xC, 0xF, false);
  v = max(v, t31);
  return __builtin_amdgcn_readlane(v, 63);
}

template <class A, bool STORE_GATES>
__device__ void select_topk(const float* logits, uint32_t E, uint32_t K, float blend, uint32_t lane,
                            void* gates_out, int& my_e, float& my_score) {
  using Key = SelectKey<A>;
  using T = typename Key::T;
  float l[kMaxExpertsPerLane];
  int lmax_key = float_order(-FLT_MAX);
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64 * m;
    l[m] = e < E ? logits[e] : -FLT_MAX;
    lmax_key = max(lmax_key, float_order(l[m]));
  }
  const float lmax = order_float(wave_max_i32(lmax_key));
  float ex[kMaxExpertsPerLane];
  float local = 0.0f;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    ex[m] = lane + 64 * m < E ? exp_neg(l[m] - lmax) : 0.0f;
    local += ex[m];
  }
  const float inv_total = 1.0f / wave_sum_all(local);
  T key[kMaxExpertsPerLane];
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64 * m;
    const float gate = A::round(ex[m] * inv_total);
    if constexpr (STORE_GATES) {
      if (e < E) A::store(gates_out, e, gate);
    }
    key[m] = e < E ? Key::make(gate, e) : T(0);
  }
  // optimal 19-comparator sorting network for 8 keys, descending
  cas_desc(key[0], key[1]); cas_desc(key[2], key[3]); cas_desc(key[4], key[5]); cas_desc(key[6], key[7]);
  cas_desc(key[0], key[2]); cas_desc(key[1], key[3]); cas_desc(key[4], key[6]); cas_desc(key[5], key[7]);
  cas_desc(key[1], key[2]); cas_desc(key[5], key[6]); cas_desc(key[0], key[4]); cas_desc(key[3], key[7]);
  cas_desc(key[1], key[5]); cas_desc(key[2], key[6]);
  cas_desc(key[1], key[4]); cas_desc(key[3], key[6]);
  cas_desc(key[2], key[4]); cas_desc(key[3], key[5]);
  cas_desc(key[3], key[4]);
  float mass = 0.0f;
  my_e = 0;
  float my_gate = 0.0f;
  for (uint32_t k = 0; k < K; ++k) {
    const T win = Key::wave_max(key[0]);
    const float g = Key::gate(win);
    mass += g;
    if (lane == k) {
      my_e = static_cast<int>(Key::expert(win));
      my_gate = g;
    }
    if (key[0] == win) {  // keys are unique: exactly one lane pops its head
#pragma unroll
      for (int m = 0; m < kMaxExpertsPerLane - 1; ++m) key[m] = key[m + 1];
      key[kMaxExpertsPerLane - 1] = T(0);
    }
  }
  // scores / (mass + blend * (selected_mass - mass)), each step rounded
  mass = A::round(mass);
  const float diff = A::round(mass - mass);
  const float normalizer = A::round(mass + A::round(blend * diff));
  my_score = A::round(my_gate / normalizer);
}

__global__ __launch_bounds__(64) void k_select_bf16(SelectLaunch p);
__global__ __launch_bounds__(64) void k_select_f32(SelectLaunch p);

template <class A>
__device__ void select_body(const SelectLaunch& p) {
  const uint32_t t = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  int e;
  float score;
  void* gates = p.gates == nullptr ? nullptr
                                   : static_cast<char*>(p.gates) + static_cast<size_t>(t) * p.experts * A::kBytes;
  const float* logits = p.logits + static_cast<size_t>(t) * p.experts;
  if (gates != nullptr) select_topk<A, true>(logits, p.experts, p.top_k, p.blend, lane, gates, e, score);
  else select_topk<A, false>(logits, p.experts, p.top_k, p.blend, lane, nullptr, e, score);
  if (lane < p.top_k) {
    p.inds[static_cast<size_t>(t) * p.top_k + lane] = e;
    A::store(p.scores, static_cast<size_t>(t) * p.top_k + lane, score);
  }
}

__global__ __launch_bounds__(64) void k_select_bf16(SelectLaunch p) { select_body<ActBF16>(p); }
__global__ __launch_bounds__(64) void k_select_f32(SelectLaunch p) { select_body<ActF32>(p); }

// -------------------------------------------------------------- front -----

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

// One router row per wave.  CH = 16-byte chunks per lane per row (hidden/512,
// rounded up).  With a single token its activations stay in registers.
template <class A, int CH>
__device__ void router_row(const FrontLaunch& p, uint32_t row, uint32_t lane) {
  const uint32_t H = p.hidden;
  uint4 w[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint32_t e8 = 8 * (lane + 64 * c);
    w[c] = e8 < H ? *reinterpret_cast<const uint4*>(p.weight + static_cast<size_t>(row) * H + e8)
                  : make_uint4(0, 0, 0, 0);
  }
  for (uint32_t t = 0; t < p.tokens; ++t) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t e8 = 8 * (lane + 64 * c);
      RouterChunk<A> xc;
      if (e8 < H) xc.load(p.x, static_cast<size_t>(t) * H + e8); else xc.zero();
      acc = xc.dot(w[c], acc);
    }
    acc = group_sum<64>(acc);
    if (lane == 63) {
      if (p.bias != nullptr) acc += p.bias[row];
      p.logits[static_cast<size_t>(t) * p.experts + row] = A::round(acc);
    }
  }
}

// The shared expert's H -> 1 quantized gate followed by the sigmoid.
template <class A>
__device__ void shared_gate_logit(const FrontLaunch& p, uint32_t lane) {
  const uint32_t H = p.hidden, G = H / kGroup;
  constexpr int GW = lds_group_words<A>();
  for (uint32_t t = 0; t < p.tokens; ++t) {
    float acc = 0.0f;
    for (uint32_t g = lane; g < G; g += 64) {
      const uint4 w = *reinterpret_cast<const uint4*>(p.seg.w + g * kWordsPerGroup);
      uint32_t buf[GW];
      stage_group<A>(p.x, static_cast<size_t>(t) * H + g * kGroup, buf);
      GroupAct<A> xa;
      xa.load_lds(buf);
      acc += xa.apply(w, bf16_to_f32(p.seg.s[g]), bf16_to_f32(p.seg.b[g]));
    }
    const float logit = A::round(wave_sum_all(acc));
    if (lane == 0) A::store(p.shared_sig, t, sigmoid_act<A>(logit));
  }
}

template <class A, int CH>
__global__ __launch_bounds__(kBlock) void k_front(FrontLaunch p, uint32_t router_blocks) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  if (blockIdx.x >= router_blocks) {
    if (wave == 0) shared_gate_logit<A>(p, lane);
  } else {
    const uint32_t row = blockIdx.x * kWaves + wave;
    if (row < p.experts) router_row<A, CH>(p, row, lane);
  }
  if (p.trace != nullptr && threadIdx.x == 0) {
    tr.mark(1);
    tr.t[2] = tr.t[3] = tr.t[4] = tr.t[1];
    tr.write(p.trace, 1, blockIdx.x);
  }
}

// ------------------------------------------------------------- gate/up ----

template <class A, int LPR, int GI, int U>
__global__ __launch_bounds__(kBlock) void k_gateup(GateUpLaunch p) {
  constexpr int RPI = 64 / LPR;
  constexpr int RPW = RPI * U;
  constexpr int RPB = RPW * kWaves;
  constexpr int GW = lds_group_words<A>();
  extern __shared__ uint4 lds_raw[];
  uint32_t* lds_x = reinterpret_cast<uint32_t*>(lds_raw);  // G * GW words
  __shared__ int s_sel[kMaxTopK];
  __shared__ float s_score[kMaxTopK];
  __shared__ int s_table[kMaxExpertsPerLane * 64];
  __shared__ float s_g[RPB], s_u[RPB];
  __shared__ uint32_t s_word, s_ok;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t lr = lane % LPR;
  const uint32_t rw = lane / LPR;
  const uint32_t pair = blockIdx.y;
  const uint32_t routed_pairs = p.tokens * p.slots;
  const bool shared_pair = pair >= routed_pairs;
  const uint32_t t = shared_pair ? pair - routed_pairs : pair / p.slots;
  const uint32_t j = shared_pair ? p.slots : pair % p.slots;
  const uint32_t S = p.slots + p.has_shared;
  const uint32_t H = p.hidden, I = p.inter, G = H / kGroup;
  const bool select = !shared_pair && p.logits != nullptr;
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);

  // prologue: expert selection (wave 0), slot table (wave 1), activations (rest)
  if (select && wave == 0) {
    int e;
    float score;
    if (p.trace != nullptr) {  // when the logits arrive
      const float first = p.logits[static_cast<size_t>(t) * p.experts + lane];
      if (first == 12345.0f) s_score[0] = first;
      tr.mark(5);
    }
    select_topk<A, false>(p.logits + static_cast<size_t>(t) * p.experts, p.experts, p.slots, p.blend, lane, nullptr, e,
                   score);
    if (p.trace != nullptr) {
      tr.mark(6);
      int e2;
      float score2;
      select_topk<A, false>(p.logits + static_cast<size_t>(t) * p.experts, p.experts, p.slots, p.blend, lane,
                            nullptr, e2, score2);
      if (e2 != e || score2 != score) s_score[0] = -1.0f;
      tr.mark(9);
    }
    if (lane < p.slots) {
      s_sel[lane] = e;
      s_score[lane] = score;
    }
  }
  if (select && wave == 1 && p.slot_table != nullptr) {
    for (uint32_t e = lane; e < p.experts; e += 64) s_table[e] = p.slot_table[e];
  }
  const uint32_t first = select ? 2 * 64 : 0;
  for (uint32_t g = tid - first; tid >= first && g < G; g += kBlock - first)
    stage_group<A>(p.x, static_cast<size_t>(t) * H + g * kGroup, lds_x + g * GW);
  if (tid == 0 && !select) {
    if (shared_pair) {
      s_ok = 1;
    } else {
      s_word = p.routes[t * p.slots + j];
      s_ok = 1;
    }
  }
  if (p.trace != nullptr) tr.mark(7);
  __syncthreads();
  if (p.trace != nullptr) tr.mark(8);
  if (select) {
    if (tid == 0) {
      const int e = s_sel[j];
      uint32_t word = static_cast<uint32_t>(e);
      if (p.slot_table != nullptr) {
        const int slot = s_table[e];
        word = slot >= 0 ? (kSlotBit | static_cast<uint32_t>(slot)) : kMissWord;
      }
      s_word = word;
    }
    // one block per token publishes the selection for the down kernel
    if (blockIdx.x == 0 && j == 0 && tid < p.slots) {
      const size_t o = static_cast<size_t>(t) * p.slots + tid;
      const int e = s_sel[tid];
      uint32_t word = static_cast<uint32_t>(e);
      if (p.slot_table != nullptr) {
        const int slot = s_table[e];
        word = slot >= 0 ? (kSlotBit | static_cast<uint32_t>(slot)) : kMissWord;
      }
      if (p.inds_out != nullptr) p.inds_out[o] = e;
      if (p.scores_out != nullptr) A::store(p.scores_out, o, s_score[tid]);
      if (p.words_out != nullptr) p.words_out[o] = word;
    }
    __syncthreads();
  }

  ProjPtrs gp{}, upp{};
  bool ok = true;
  if (shared_pair) {
    gp = p.shared_gate;
    upp = p.shared_up;
  } else {
    const uint32_t word = s_word;
    const int32_t* table = select ? nullptr : p.slot_table;
    ok = resolve_proj(word, table, p.experts, p.pool, p.gate, 0, I, H, gp, &p.stream) &&
         resolve_proj(word, table, p.experts, p.pool, p.up, 1, I, H, upp, &p.stream);
  }
  if (!ok && tid == 0 && blockIdx.x == 0) flag(p.status, 1u);
  if (p.trace != nullptr) tr.mark(1);

  const uint32_t row_base = blockIdx.x * RPB + wave * RPW + rw;
  uint4 wg[U][GI], wu[U][GI];
  uint32_t sg[U][GI], bg[U][GI], su[U][GI], bu[U][GI];
  const size_t row_words = H / 8;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t row = row_base + u * RPI;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      const uint32_t g = lr + it * LPR;
      if (ok && row < I && g < G) {
        const size_t wo = row * row_words + g * kWordsPerGroup;
        const size_t mo = static_cast<size_t>(row) * G + g;
        wg[u][it] = *reinterpret_cast<const uint4*>(gp.w + wo);
        wu[u][it] = *reinterpret_cast<const uint4*>(upp.w + wo);
        sg[u][it] = gp.s[mo];
        bg[u][it] = gp.b[mo];
        su[u][it] = upp.s[mo];
        bu[u][it] = upp.b[mo];
      } else {
        wg[u][it] = wu[u][it] = make_uint4(0, 0, 0, 0);
        sg[u][it] = bg[u][it] = su[u][it] = bu[u][it] = 0;
      }
    }
  }
  GroupAct<A> xa[GI];
#pragma unroll
  for (int it = 0; it < GI; ++it) {
    const uint32_t g = lr + it * LPR;
    xa[it].load_lds(lds_x + (g < G ? g : 0) * GW);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      if (lr + it * LPR < G) {
        ag += xa[it].apply(wg[u][it], bf16_to_f32(sg[u][it]), bf16_to_f32(bg[u][it]));
        au += xa[it].apply(wu[u][it], bf16_to_f32(su[u][it]), bf16_to_f32(bu[u][it]));
      }
    }
    ag = group_sum<LPR>(ag);
    au = group_sum<LPR>(au);
    if (lr == LPR - 1) {
      const uint32_t r = wave * RPW + rw + u * RPI;
      s_g[r] = ag;
      s_u[r] = au;
    }
    if (u == 0 && p.trace != nullptr) tr.mark(2);
  }
  if (p.trace != nullptr) tr.mark(3);
  __syncthreads();
  // block-parallel epilogue: one thread per row
  if (tid < RPB) {
    const uint32_t row = blockIdx.x * RPB + (tid / RPW) * RPW + tid % RPW;
    if (row < I) {
      const float gv = A::round(s_g[tid]);
      const float uv = A::round(s_u[tid]);
      const size_t act_base = (static_cast<size_t>(t) * S + j) * I;
      A::store(p.act, act_base + row, ok ? swiglu_act<A>(gv, uv) : 0.0f);
      if (!shared_pair) {
        const size_t o = (static_cast<size_t>(t) * p.slots + j) * I + row;
        if (p.gate_out != nullptr) A::store(p.gate_out, o, gv);
        if (p.up_out != nullptr) A::store(p.up_out, o, uv);
      }
    }
  }
  if (p.trace != nullptr && tid == 0) {
    tr.mark(4);
    tr.write(p.trace, select ? 2 : 3, blockIdx.y * gridDim.x + blockIdx.x);
  }
}

// ----------------------------------------------------------------- down ---

constexpr int kDownMaxSlots = 12;  // MAX_TOP_K (10) + shared, rounded up
constexpr int kDownQuads = 2;      // row groups of 64/LPR rows per block
constexpr int kDownMaxUnits = (kDownMaxSlots * kDownQuads + kWaves - 1) / kWaves;

template <class A, int LPR>
__global__ __launch_bounds__(kBlock) void k_down(DownLaunch p) {
  constexpr int RPI = 64 / LPR;
  constexpr int RB = RPI * kDownQuads;
  constexpr int GW = lds_group_words<A>();
  extern __shared__ uint4 lds_raw[];
  uint32_t* lds_act = reinterpret_cast<uint32_t*>(lds_raw);
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

  // 1. lane k < K resolves slot k once (one load latency for all slots), the
  //    units take their pointers with readlane and issue their weight loads
  ProjPtrs mine{};
  bool mine_ok = false;
  if (lane < K) {
    mine_ok = resolve_proj(p.routes[t * K + lane], p.slot_table, p.experts, p.pool, p.down, 2, H, I, mine,
                           &p.stream);
    if (!mine_ok && wave == 0 && blockIdx.x == 0) flag(p.status, 1u);
  }
  const uint64_t ok_mask = __ballot(mine_ok);
  if (p.trace != nullptr) tr.mark(5);
  uint4 w[kDownMaxUnits];
  uint32_t sc[kDownMaxUnits], bi[kDownMaxUnits];
  const size_t row_words = I / 8;
#pragma unroll
  for (int i = 0; i < kDownMaxUnits; ++i) {
    const uint32_t unit = wave + kWaves * i;
    const uint32_t slot = unit / kDownQuads;
    const uint32_t quad = unit % kDownQuads;
    const uint32_t row = row0 + quad * RPI + rw;
    ProjPtrs dp{};
    bool ok = false;
    if (unit < S * kDownQuads) {
      if (slot < K) {
        ok = (ok_mask >> slot) & 1u;
        dp.w = reinterpret_cast<const uint32_t*>(readlane_u64(reinterpret_cast<uint64_t>(mine.w), slot));
        dp.s = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mine.s), slot));
        dp.b = reinterpret_cast<const uint16_t*>(readlane_u64(reinterpret_cast<uint64_t>(mine.b), slot));
      } else {
        dp = p.shared_down;
        ok = true;
      }
    }
    if (ok && row < H && lr < G) {
      w[i] = *reinterpret_cast<const uint4*>(dp.w + row * row_words + lr * kWordsPerGroup);
      sc[i] = dp.s[static_cast<size_t>(row) * G + lr];
      bi[i] = dp.b[static_cast<size_t>(row) * G + lr];
    } else {
      w[i] = make_uint4(0, 0, 0, 0);
      sc[i] = bi[i] = 0;
    }
  }
  if (p.trace != nullptr) tr.mark(6);

  // 2. stage the token's activations (all slots) into LDS; prefetch the epilogue operands
  for (uint32_t item = tid; item < S * G; item += kBlock) {
    const uint32_t slot = item / G, g = item % G;
    stage_group<A>(p.act, (static_cast<size_t>(t) * S + slot) * I + g * kGroup, lds_act + item * GW);
  }
  if (p.trace != nullptr) tr.mark(7);
  if (p.scores != nullptr) {
    if (tid < K) s_scores[tid] = load_any(p.scores, static_cast<size_t>(t) * K + tid, p.score_dtype);
    const uint32_t r = tid - 64;  // wave 1 prefetches the shared term of the tile
    if (tid >= 64 && r < RB && row0 + r < H) {
      const size_t o = static_cast<size_t>(t) * H + row0 + r;
      if (p.shared_y != nullptr) s_shared[r] = A::load(p.shared_y, o);
      else if (p.shared != nullptr) s_shared[r] = A::load(p.shared, o);
    }
    if (tid == 128) {
      if (p.has_shared) s_sig = A::load(p.shared_sig, t);
      else if (p.shared != nullptr) s_sig = A::load(p.shared_gate, t);
    }
  }
  if (p.trace != nullptr) tr.mark(8);
  __syncthreads();
  if (p.trace != nullptr) tr.mark(1);

  // 3. dot products, row sums, partials to LDS
#pragma unroll
  for (int i = 0; i < kDownMaxUnits; ++i) {
    const uint32_t unit = wave + kWaves * i;
    if (unit >= S * kDownQuads) break;  // wave-uniform
    const uint32_t slot = unit / kDownQuads;
    const uint32_t quad = unit % kDownQuads;
    float v = 0.0f;
    if (lr < G) {
      GroupAct<A> xa;
      xa.load_lds(lds_act + (slot * G + lr) * GW);
      v = xa.apply(w[i], bf16_to_f32(sc[i]), bf16_to_f32(bi[i]));
    }
    v = group_sum<LPR>(v);
    if (lr == LPR - 1) s_part[slot * RB + quad * RPI + rw] = v;
    if (i == 0 && p.trace != nullptr) tr.mark(2);
  }
  if (p.trace != nullptr) tr.mark(3);
  __syncthreads();

  // 4. epilogue
  if (p.scores != nullptr) {
    if (tid < RB && row0 + tid < H) {
      const uint32_t r = tid;
      float combined = 0.0f;
      for (uint32_t k = 0; k < K; ++k)
        combined = __fadd_rn(combined, __fmul_rn(A::round(s_part[k * RB + r]), s_scores[k]));
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
    }
  } else {
    for (uint32_t idx = tid; idx < K * RB; idx += kBlock) {
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

template <class K>
hipError_t ensure_lds(K* kernel, size_t bytes, size_t& granted) {
  if (bytes > granted) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return e;
    granted = bytes;
  }
  return hipSuccess;
}

template <class A, int LPR, int GI, int U>
hipError_t gateup_go(const GateUpLaunch& p, hipStream_t stream) {
  constexpr int RPB = (64 / LPR) * U * kWaves;
  const uint32_t pairs = p.tokens * p.slots + (p.has_shared ? p.tokens : 0);
  const size_t lds = static_cast<size_t>(p.hidden / kGroup) * lds_group_words<A>() * 4;
  static size_t granted = 48 * 1024;
  hipError_t e = ensure_lds(&k_gateup<A, LPR, GI, U>, lds, granted);
  if (e != hipSuccess) return e;
  dim3 grid((p.inter + RPB - 1) / RPB, pairs);
  GateUpLaunch q = p;
  q.trace = trace_reserve(grid.x * grid.y);
  hipLaunchKernelGGL((k_gateup<A, LPR, GI, U>), grid, dim3(kBlock), lds, stream, q);
  return hipGetLastError();
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
  if (gi <= 1) return gateup_go<A, 64, 1, 2>(p, stream);
  if (gi <= 2) return gateup_go<A, 64, 2, 2>(p, stream);
  return gateup_go<A, 64, 4, 1>(p, stream);
}

template <class A>
size_t down_lds_bytes(uint32_t slots_total, uint32_t inter) {
  return static_cast<size_t>(slots_total) * (inter / kGroup) * lds_group_words<A>() * 4;
}

template <class A, int LPR>
hipError_t down_go(const DownLaunch& p, hipStream_t stream) {
  constexpr int RB = (64 / LPR) * kDownQuads;
  const size_t lds = down_lds_bytes<A>(p.slots + p.has_shared, p.inter);
  static size_t granted = 48 * 1024;
  hipError_t e = ensure_lds(&k_down<A, LPR>, lds, granted);
  if (e != hipSuccess) return e;
  dim3 grid((p.hidden + RB - 1) / RB, p.tokens);
  DownLaunch q = p;
  q.trace = trace_reserve(grid.x * grid.y);
  hipLaunchKernelGGL((k_down<A, LPR>), grid, dim3(kBlock), lds, stream, q);
  return hipGetLastError();
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
void front_go(const FrontLaunch& p0, hipStream_t stream) {
  const uint32_t router_blocks = (p0.experts + kWaves - 1) / kWaves;
  const uint32_t blocks = router_blocks + (p0.seg.w != nullptr ? 1 : 0);
  FrontLaunch p = p0;
  p.trace = trace_reserve(blocks);
  const uint32_t chunks = (p.hidden / 8 + 63) / 64;
  if (chunks <= 1) hipLaunchKernelGGL((k_front<A, 1>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else if (chunks <= 2) hipLaunchKernelGGL((k_front<A, 2>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else if (chunks <= 4) hipLaunchKernelGGL((k_front<A, 4>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else if (chunks <= 8) hipLaunchKernelGGL((k_front<A, 8>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else hipLaunchKernelGGL((k_front<A, 16>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
}

}  // namespace

bool gateup_supported(uint32_t hidden) {
  return hidden % kGroup == 0 && hidden > 0 && hidden / kGroup <= 256;
}

bool down_supported(uint32_t inter, uint32_t slots_total, int act_dtype) {
  if (inter % kGroup != 0 || inter == 0 || inter / kGroup > 64) return false;
  if (slots_total > static_cast<uint32_t>(kDownMaxSlots) || slots_total == 0) return false;
  const size_t lds = act_dtype == 0 ? down_lds_bytes<ActBF16>(slots_total, inter)
                                    : down_lds_bytes<ActF32>(slots_total, inter);
  return lds <= 128 * 1024;
}

hipError_t launch_front(const FrontLaunch& p, hipStream_t stream) {
  timing_begin("router", stream);
  if (p.act_dtype == 0) front_go<ActBF16>(p, stream); else front_go<ActF32>(p, stream);
  hipError_t e = hipGetLastError();
  timing_end("router", stream);
  return e;
}

hipError_t launch_select(const SelectLaunch& p, hipStream_t stream) {
  timing_begin("select", stream);
  if (p.act_dtype == 0) hipLaunchKernelGGL(k_select_bf16, dim3(p.tokens), dim3(64), 0, stream, p);
  else hipLaunchKernelGGL(k_select_f32, dim3(p.tokens), dim3(64), 0, stream, p);
  hipError_t e = hipGetLastError();
  timing_end("select", stream);
  return e;
}

hipError_t launch_gateup(const GateUpLaunch& p, hipStream_t stream) {
  timing_begin("gateup", stream);
  hipError_t e = p.act_dtype == 0 ? gateup_dispatch<ActBF16>(p, stream) : gateup_dispatch<ActF32>(p, stream);
  timing_end("gateup", stream);
  return e;
}

hipError_t launch_down(const DownLaunch& p, hipStream_t stream) {
  timing_begin("down", stream);
  hipError_t e = p.act_dtype == 0 ? down_dispatch<ActBF16>(p, stream) : down_dispatch<ActF32>(p, stream);
  timing_end("down", stream);
  return e;
}

hipError_t launch_weighted_combine(const void* values, const void* scores, void* out, uint32_t tokens,
                                   uint32_t slots, uint32_t hidden, int act_dtype, int score_dtype,
                                   hipStream_t stream) {
  const size_t n = static_cast<size_t>(tokens) * hidden;
  const uint32_t blocks = static_cast<uint32_t>((n + kBlock - 1) / kBlock);
  timing_begin("combine", stream);
  if (act_dtype == 0) {
    hipLaunchKernelGGL(k_weighted_combine<ActBF16>, dim3(blocks), dim3(kBlock), 0, stream, values, scores, out,
                       tokens, slots, hidden, score_dtype);
  } else {
    hipLaunchKernelGGL(k_weighted_combine<ActF32>, dim3(blocks), dim3(kBlock), 0, stream, values, scores, out,
                       tokens, slots, hidden, score_dtype);
  }
  hipError_t e = hipGetLastError();
  timing_end("combine", stream);
  return e;
}

}  // namespace vm
